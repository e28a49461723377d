"""Single-token decode with the chunk partials merged inside the split launch
(MI_ATTN_DECODE_MERGE=1: XCD-local merge through L2, then across XCDs),
against the CPU oracle (reference math of src/math_util.rs:264-269, 323-383)
and against the default two-launch path, through the C ABI.  The merge's
counters are reset by the kernels themselves, so calls of every size follow
each other and graph replays repeat."""
import numpy as np
import pytest
import torch

from moe_infer_amd import Cache, attn_decode, attn_step, attn_step_proj
from oracle import oracle as O

from .conftest import f16
from .gpu_util import announce, assert_close, dev, host

pytestmark = pytest.mark.gpu
H, G, D = 16, 2, 256


@pytest.fixture(autouse=True)
def merged(monkeypatch):
    monkeypatch.setenv("MI_ATTN_DECODE_MERGE", "1")


def filled_cache(k, v, capacity=None):
    L = k.shape[0]
    c = Cache(num_layers=1, capacity=capacity or max(L, 1))
    if L:
        c.upload(0, k, v)
        c.set_pos(L)
    return c


@pytest.mark.parametrize("L", [1, 7, 33, 256, 257, 2000, 4099, 8193, 32768, 40000])
@pytest.mark.parametrize("gated", [False, True])
def test_merged_decode_matches_oracle(L, gated):
    announce(f"merged decode L={L} gated={gated}")
    rng = np.random.default_rng(500 + L)
    q, k, v, g = f16(rng, H * D), f16(rng, L, G * D), f16(rng, L, G * D), f16(rng, H * D)
    c = filled_cache(k, v)
    out = attn_decode(c, 0, dev(q), L, gate=dev(g) if gated else None)
    assert_close(out, O.decode(q, k, v, L, gate=g if gated else None), f"merged decode L={L}")


def test_merged_calls_of_every_size_in_a_row_and_against_two_launches(monkeypatch):
    """Lengths from 1 to 4 chunks per XCD and back, each call against the
    oracle and against the two-launch path on the same inputs (the
    counters of each call start at zero)."""
    rng = np.random.default_rng(41)
    Lmax = 33000
    k, v = f16(rng, Lmax, G * D), f16(rng, Lmax, G * D)
    c = filled_cache(k, v)
    for L in [33000, 1, 300, 9000, 33, 32768, 2, 5000]:
        announce(f"merged decode sequence L={L}")
        q, g = f16(rng, H * D), f16(rng, H * D)
        monkeypatch.setenv("MI_ATTN_DECODE_MERGE", "1")
        out = host(attn_decode(c, 0, dev(q), L, gate=dev(g)))
        monkeypatch.setenv("MI_ATTN_DECODE_MERGE", "0")
        two = host(attn_decode(c, 0, dev(q), L, gate=dev(g)))
        assert_close(out, O.decode(q, k[:L], v[:L], L, gate=g), f"merged L={L}")
        assert_close(out, two, f"merged vs two launches L={L}", atol=1e-4)


def test_merged_seq_len_zero_and_poisoned_tail():
    announce("merged decode L=0 / poisoned tail")
    rng = np.random.default_rng(42)
    L, P = 45, 300
    k, v, q = f16(rng, P, G * D), f16(rng, P, G * D), f16(rng, H * D)
    k[L:] = np.float16(np.nan)
    v[L:] = np.float16(np.inf)
    c = filled_cache(k, v)
    assert torch.count_nonzero(attn_decode(c, 0, dev(q), 0)).item() == 0
    assert_close(attn_decode(c, 0, dev(q), L), O.decode(q, k[:L], v[:L], L),
                 "merged decode poisoned tail")


def test_merged_step_sequence():
    """append-then-attend token by token (cpu.rs:141-167) through the merged
    step, with the cache growing across 256 rows."""
    announce("merged attn_step sequence")
    rng = np.random.default_rng(43)
    T = 280
    c = Cache(num_layers=1, capacity=16)
    ks, vs = f16(rng, T, G * D), f16(rng, T, G * D)
    for t in range(T):
        q, g = f16(rng, H * D), f16(rng, H * D)
        out = attn_step(c, 0, dev(q), dev(ks[t]), dev(vs[t]), t, gate=dev(g))
        if t % 31 == 0 or t in (255, 256, T - 1):
            assert_close(out, O.decode(q, ks[:t + 1], vs[:t + 1], t + 1, gate=g),
                         f"merged step t={t}")
        c.set_pos(t + 1)


def test_merged_graph_replay_matches_eager(monkeypatch):
    """The merged step and step-from-projections captured in one HIP graph;
    four replays with eager work between them equal the eager outputs bit
    for bit, and the eager outputs equal the two-launch path's."""
    announce("merged graph replay")
    rng = np.random.default_rng(44)
    L = 20000
    k, v = f16(rng, L + 4, G * D), f16(rng, L + 4, G * D)
    c = filled_cache(k[:L], v[:L], capacity=L + 64)
    q, g = dev(f16(rng, H * D)), dev(f16(rng, H * D))
    kn, vn = dev(k[L]), dev(v[L])
    qp = torch.from_numpy(rng.standard_normal((H, 2 * D)).astype(np.float32)).cuda()
    kp = torch.from_numpy(rng.standard_normal((G, D)).astype(np.float32)).cuda()
    vp = torch.from_numpy(rng.standard_normal((G, D)).astype(np.float32)).cuda()
    qw = torch.ones(D, dtype=torch.bfloat16, device="cuda")
    out1 = torch.empty(H * D, dtype=torch.float16, device="cuda")
    out2 = torch.empty(H, D, dtype=torch.float16, device="cuda")

    def step():
        attn_step(c, 0, q, kn, vn, L, gate=g, out=out1)
        attn_step_proj(c, 0, qp, kp, vp, qw, qw, L + 1, out=out2)

    step()
    torch.cuda.synchronize()
    ref = [out1.clone(), out2.clone()]
    monkeypatch.setenv("MI_ATTN_DECODE_MERGE", "0")
    step()
    torch.cuda.synchronize()
    assert_close(out1, host(ref[0]), "merged step vs two launches", atol=1e-4)
    assert_close(out2, host(ref[1]), "merged step_proj vs two launches", atol=1e-4)
    monkeypatch.setenv("MI_ATTN_DECODE_MERGE", "1")
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    other = filled_cache(k[:300], v[:300])
    for r in range(4):
        out1.fill_(7.0)
        out2.fill_(7.0)
        graph.replay()
        attn_decode(other, 0, q, 300)  # eager merged work between the replays
        torch.cuda.synchronize()
        assert torch.equal(ref[0].view(torch.int16), out1.view(torch.int16)), f"replay {r}"
        assert torch.equal(ref[1].view(torch.int16), out2.view(torch.int16)), f"replay {r}"
    assert_close(out1, O.decode(host(q), k[:L + 1], v[:L + 1], L + 1, gate=host(g)),
                 "merged graph step vs oracle")

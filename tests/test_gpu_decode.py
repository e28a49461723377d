"""Decode, engine step and K-token verify on the GPU against the CPU oracle
(reference f32 math of src/math_util.rs:264-269, 323-383 on the same f16
inputs), through the C ABI."""
import warnings

import numpy as np
import pytest
import torch

from moe_infer_amd import Cache, attn_decode, attn_step, attn_verify
from oracle import oracle as O

from .conftest import f16
from .gpu_util import announce, assert_close, dev, host

pytestmark = pytest.mark.gpu
H, G, D = 16, 2, 256


def filled_cache(k, v, capacity=None):
    L = k.shape[0]
    c = Cache(num_layers=1, capacity=capacity or max(L, 1))
    if L:
        c.upload(0, k, v)
        c.set_pos(L)
    return c


@pytest.mark.parametrize("L", [1, 2, 7, 31, 32, 33, 255, 256, 257, 512, 1000, 4099])
@pytest.mark.parametrize("gated", [False, True])
def test_decode_matches_oracle(L, gated):
    announce(f"decode L={L} gated={gated}")
    rng = np.random.default_rng(100 + L)
    q, k, v, g = f16(rng, H * D), f16(rng, L, G * D), f16(rng, L, G * D), f16(rng, H * D)
    c = filled_cache(k, v)
    out = attn_decode(c, 0, dev(q), L, gate=dev(g) if gated else None)
    ref = O.decode(q, k, v, L, gate=g if gated else None)
    assert_close(out, ref, f"decode L={L}")


def test_decode_ctx32k_matches_oracle():
    """batch 1, context 32768, seed 2."""
    announce("decode C2 L=32768")
    L = 32768
    rng = np.random.default_rng(2)
    q, k, v = f16(rng, H * D), f16(rng, L, G * D), f16(rng, L, G * D)
    c = filled_cache(k, v)
    out = attn_decode(c, 0, dev(q), L)
    assert_close(out, O.decode(q, k, v, L), "decode L=32768 vs f32 oracle")
    assert_close(out, O.decode_f64(q, k, v, L), "decode L=32768 vs f64 oracle")


def test_decode_quarter_million_rows():
    """262161 rows (chunks of 1152 keys, 228 per head): the long-context
    chunking against the oracle."""
    announce("decode L=262161")
    L = 262161
    rng = np.random.default_rng(262)
    q, g = f16(rng, H * D), f16(rng, H * D)
    k, v = f16(rng, L, G * D), f16(rng, L, G * D)
    c = filled_cache(k, v)
    out = attn_decode(c, 0, dev(q), L, gate=dev(g))
    assert_close(out, O.decode(q, k, v, L, gate=g), "decode L=262161")


def test_decode_seq_len_zero_and_bounds():
    announce("decode L=0 / bounds")
    rng = np.random.default_rng(5)
    c = filled_cache(f16(rng, 8, G * D), f16(rng, 8, G * D))
    q = dev(f16(rng, H * D))
    out = attn_decode(c, 0, q, 0)
    assert torch.count_nonzero(out).item() == 0
    with pytest.raises(ValueError):
        attn_decode(c, 0, q, c.capacity + 1)


def test_decode_never_reads_rows_past_seq_len():
    """Rows past seq_len (stale after rollback) are never read: poison them
    with NaN/inf and the output must equal the oracle on the valid rows."""
    announce("decode poisoned tail")
    rng = np.random.default_rng(6)
    L, P = 45, 300
    k, v, q = f16(rng, P, G * D), f16(rng, P, G * D), f16(rng, H * D)
    k[L:] = np.float16(np.nan)
    v[L:] = np.float16(np.inf)
    c = filled_cache(k, v)
    out = attn_decode(c, 0, dev(q), L)
    assert_close(out, O.decode(q, k[:L], v[:L], L), "decode poisoned tail")


def test_engine_step_sequence():
    """append-then-attend token by token (cpu.rs:141-167): token t attends
    rows [0, t] including its own row."""
    announce("attn_step sequence")
    rng = np.random.default_rng(9)
    T = 300
    c = Cache(num_layers=2, capacity=16)  # 256 rows: grows by doubling at t = 256
    ks, vs = f16(rng, T, G * D), f16(rng, T, G * D)
    for t in range(T):
        q, g = f16(rng, H * D), f16(rng, H * D)
        for layer in (0, 1):
            out = attn_step(c, layer, dev(q), dev(ks[t]), dev(vs[t]), t, gate=dev(g))
            if t % 37 == 0 or t in (255, 256, T - 1):
                assert_close(out, O.decode(q, ks[:t + 1], vs[:t + 1], t + 1, gate=g),
                             f"step t={t} layer={layer}")
        assert c.len(0) == t + 1
        c.set_pos(t + 1)
    assert c.capacity >= T


@pytest.mark.parametrize("n,past", [(1, 0), (2, 5), (3, 31), (4, 61), (4, 255), (7, 100),
                                    (9, 1000), (6, 20000), (16, 0), (5, 59), (16, 61),
                                    (13, 4093), (12, 4096), (16, 20000), (17, 0), (33, 100),
                                    (40, 5000)])
def test_verify_matches_causal_oracle(n, past):
    announce(f"verify n={n} past={past}")
    rng = np.random.default_rng(1000 * n + past)
    kp, vp = f16(rng, past, G * D), f16(rng, past, G * D)
    q, k, v, g = f16(rng, n, H, D), f16(rng, n, G * D), f16(rng, n, G * D), f16(rng, n, H, D)
    c = filled_cache(kp, vp, capacity=past + n)
    out = attn_verify(c, 0, dev(q), dev(k), dev(v), past, gate=dev(g))
    ref = O.causal(q, np.concatenate([kp, k]), np.concatenate([vp, v]), past, gate=g)
    assert_close(out, ref, f"verify n={n} past={past}")
    assert c.len(0) == past + n


@pytest.mark.parametrize("n,past", [(16, 20000), (8, 20000)])
def test_wide_verify_rising_scores_and_grouped_form(n, past, monkeypatch):
    """5..16 tokens run the wide verify (the prefill's MFMA tiles over key
    chunks of a few 64-key tiles).  Keys whose scores rise steeply along the
    context put a chunk's later tiles far above its first tile's max (the
    fixed reference max), so the workgroups take the restart path; the
    result matches the oracle and the grouped 4-token form
    (MI_ATTN_VERIFY_WIDE=0)."""
    announce(f"wide verify rising n={n} past={past}")
    rng = np.random.default_rng(n + past)
    L = past + n
    q = f16(rng, n, H, D)
    qdir = q[0].astype(np.float32).reshape(G, 8, D)[:, 0]  # token 0, head 0 of each group
    qdir /= np.linalg.norm(qdir, axis=-1, keepdims=True)
    # for those rows, odd 64-key tiles score ~30 (base 2) above even ones: a
    # chunk that starts on an even tile meets keys far above its first
    # tile's max
    ramp = ((np.arange(L) // 64) % 2).astype(np.float32)[:, None, None] * 21.0
    kall = (0.3 * rng.standard_normal((L, G, D)).astype(np.float32) + ramp * qdir[None])
    kall = kall.astype(np.float16).reshape(L, G * D)
    vall = f16(rng, L, G * D)
    g = f16(rng, n, H, D)
    # scores (base 2) of the first row: odd tiles far above even ones
    s2 = (kall[:, :D].astype(np.float32) @ q[0, 0].astype(np.float32)) / 16 * 1.4427
    assert s2[64:128].min() - s2[:64].max() > 15
    c = filled_cache(kall[:past], vall[:past], capacity=L)
    out = attn_verify(c, 0, dev(q), dev(kall[past:]), dev(vall[past:]), past, gate=dev(g))
    ref = O.causal(q, kall, vall, past, gate=g)
    assert_close(out, ref, f"wide verify rising n={n}")
    monkeypatch.setenv("MI_ATTN_VERIFY_WIDE", "0")
    c.set_pos(past)
    grouped = attn_verify(c, 0, dev(q), dev(kall[past:]), dev(vall[past:]), past, gate=dev(g))
    assert_close(grouped, ref, f"grouped verify rising n={n}")


def test_verify_c5_and_rollback():
    """K=4 drafts appended to a 65536-row cache, causal
    within the drafts, sigmoid gate; then rollback to 65538: rows below are
    unchanged, len == 65538, and the next append lands at 65538."""
    announce("verify C5 65536+4 and rollback")
    rng = np.random.default_rng(5)
    P, K = 65536, 4
    kp, vp = f16(rng, P, G * D), f16(rng, P, G * D)
    q, k, v, g = f16(rng, K, H, D), f16(rng, K, G * D), f16(rng, K, G * D), f16(rng, K, H, D)
    c = filled_cache(kp, vp, capacity=P + K)
    out = attn_verify(c, 0, dev(q), dev(k), dev(v), P, gate=dev(g))
    kall, vall = np.concatenate([kp, k]), np.concatenate([vp, v])
    assert_close(out, O.causal(q, kall, vall, P, gate=g), "verify C5")
    c.set_pos(P + 2)
    assert c.pos == P + 2 and c.len(0) == P + 2
    kd, vd = c.download(0, rows=P + K)
    assert np.array_equal(kd.view(np.uint16), kall.view(np.uint16))
    assert np.array_equal(vd.view(np.uint16), vall.view(np.uint16))
    # the accepted prefix decodes like a fresh cache of P+2 rows
    q2, k2, v2 = f16(rng, H * D), f16(rng, G * D), f16(rng, G * D)
    out2 = attn_step(c, 0, dev(q2), dev(k2), dev(v2), P + 2)
    kref = np.concatenate([kall[:P + 2], k2[None]])
    vref = np.concatenate([vall[:P + 2], v2[None]])
    assert_close(out2, O.decode(q2, kref, vref, P + 3), "decode after rollback")
    kd, vd = c.download(0, rows=P + K)
    assert np.array_equal(kd[P + 2].view(np.uint16), k2.view(np.uint16))
    assert np.array_equal(kd[P + 3].view(np.uint16), k[3].view(np.uint16))  # stale, untouched
    assert np.array_equal(vd[:P + 2].view(np.uint16), vall[:P + 2].view(np.uint16))


@pytest.mark.parametrize("L", [8193, 40000])
def test_decode_long_contexts(L):
    """Chunkings past the 128-key minimum (chunk 256 at 40000 rows)."""
    announce(f"decode L={L}")
    rng = np.random.default_rng(L)
    q, k, v, g = f16(rng, H * D), f16(rng, L, G * D), f16(rng, L, G * D), f16(rng, H * D)
    c = filled_cache(k, v)
    out = attn_decode(c, 0, dev(q), L, gate=dev(g))
    assert_close(out, O.decode(q, k, v, L, gate=g), f"decode L={L}")


def test_step_sequence_long_context():
    """The engine step (append fused into the split kernel) over 200 tokens
    past 8050 rows, where the number of chunks passes 64."""
    announce("step sequence at 8K")
    rng = np.random.default_rng(12)
    P = 8050
    kp, vp = f16(rng, P, G * D), f16(rng, P, G * D)
    c = filled_cache(kp, vp, capacity=P + 300)
    ks, vs = [kp], [vp]
    for t in range(P, P + 200):
        q, g, kn, vn = f16(rng, H * D), f16(rng, H * D), f16(rng, G * D), f16(rng, G * D)
        out = attn_step(c, 0, dev(q), dev(kn), dev(vn), t, gate=dev(g))
        ks.append(kn[None])
        vs.append(vn[None])
        c.set_pos(t + 1)
        if t % 50 == 0 or t == P + 199:
            assert_close(out, O.decode(q, np.concatenate(ks), np.concatenate(vs), t + 1, gate=g),
                         f"step t={t}")


def test_graph_replay_of_steps_matches_eager():
    """The engine step, the verify call and the step from projections
    captured in one HIP graph (no allocation or memset inside the library
    calls once the workspace exists); every replay, with eager work and host
    synchronisations between replays, equals the eager outputs bit for bit."""
    from moe_infer_amd import attn_step_proj
    announce("graph replay of step / verify / step_proj")
    rng = np.random.default_rng(31)
    L = 5000
    k, v = f16(rng, L + 8, G * D), f16(rng, L + 8, G * D)
    c = filled_cache(k[:L], v[:L], capacity=L + 64)
    q, g = dev(f16(rng, H * D)), dev(f16(rng, H * D))
    kn, vn = dev(k[L]), dev(v[L])
    q4, g4 = dev(f16(rng, 4, H, D)), dev(f16(rng, 4, H, D))
    k4, v4 = dev(k[L + 1:L + 5]), dev(v[L + 1:L + 5])
    qp = torch.from_numpy(rng.standard_normal((H, 2 * D)).astype(np.float32)).cuda()
    kp = torch.from_numpy(rng.standard_normal((G, D)).astype(np.float32)).cuda()
    vp = torch.from_numpy(rng.standard_normal((G, D)).astype(np.float32)).cuda()
    qw = torch.ones(D, dtype=torch.bfloat16, device="cuda")
    out1 = torch.empty(H * D, dtype=torch.float16, device="cuda")
    out4 = torch.empty(4, H, D, dtype=torch.float16, device="cuda")
    out3 = torch.empty(H, D, dtype=torch.float16, device="cuda")

    def step():
        attn_step(c, 0, q, kn, vn, L, gate=g, out=out1)
        attn_verify(c, 0, q4, k4, v4, L + 1, gate=g4, out=out4)
        attn_step_proj(c, 0, qp, kp, vp, qw, qw, L + 5, out=out3)

    step()  # eager: sizes the workspace, sets the kernels' LDS limits
    torch.cuda.synchronize()
    ref = [out1.clone(), out4.clone(), out3.clone()]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    other = filled_cache(k[:300], v[:300])
    for r in range(4):
        for o in (out1, out4, out3):
            o.fill_(7.0)
        graph.replay()
        attn_decode(other, 0, q, 300)  # eager work between the replays
        torch.cuda.synchronize()
        for a, b in zip(ref, (out1, out4, out3)):
            assert torch.equal(a.view(torch.int16), b.view(torch.int16)), f"replay {r}"
    assert_close(out1, O.decode(host(q), k[:L + 1], v[:L + 1], L + 1, gate=host(g)),
                 "graph step vs oracle")


def test_graph_replay_of_wide_verify_and_split_prefill():
    """The wide verify (8 tokens) and the split-K prefill (40 tokens after a
    past of 6008 rows), each an append, a split pass and a merge, captured in
    one HIP graph after an eager call sized the workspace: every replay, with
    eager work between, equals the eager outputs bit for bit, and those match
    the oracle."""
    from moe_infer_amd import attn_prefill
    announce("graph replay of wide verify / split-K prefill")
    rng = np.random.default_rng(33)
    L, n8, n40 = 6000, 8, 40
    k, v = f16(rng, L + n8 + n40, G * D), f16(rng, L + n8 + n40, G * D)
    c = filled_cache(k[:L], v[:L], capacity=L + n8 + n40)
    q8, g8 = dev(f16(rng, n8, H, D)), dev(f16(rng, n8, H, D))
    q40 = dev(f16(rng, n40, H, D))
    k8, v8 = dev(k[L:L + n8]), dev(v[L:L + n8])
    k40, v40 = dev(k[L + n8:]), dev(v[L + n8:])
    o8 = torch.empty(n8, H, D, dtype=torch.float16, device="cuda")
    o40 = torch.empty(n40, H, D, dtype=torch.float16, device="cuda")

    def step():
        attn_verify(c, 0, q8, k8, v8, L, gate=g8, out=o8)
        attn_prefill(c, 0, q40, k40, v40, L + n8, out=o40)

    step()  # eager: sizes the workspace, sets the kernels' LDS limits
    torch.cuda.synchronize()
    ref = [o8.clone(), o40.clone()]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    other = filled_cache(k[:300], v[:300])
    for r in range(4):
        for o in (o8, o40):
            o.fill_(7.0)
        graph.replay()
        attn_decode(other, 0, q8[0], 300)  # eager work between the replays
        torch.cuda.synchronize()
        for a, b in zip(ref, (o8, o40)):
            assert torch.equal(a.view(torch.int16), b.view(torch.int16)), f"replay {r}"
    assert_close(o8, O.causal(host(q8), k[:L + n8], v[:L + n8], L, gate=host(g8)),
                 "graph wide verify vs oracle")
    assert_close(o40, O.causal(host(q40), k, v, L + n8), "graph split-K prefill vs oracle")


def test_graph_survives_workspace_growth_on_the_same_handle():
    """A graph captured at a short context keeps replaying correctly after an
    eager call on the same handle grows its split-K workspace (the old
    workspace is kept, not freed); a call that would grow the workspace or
    the cache while the stream is capturing is refused with a ValueError."""
    from moe_infer_amd import _lib
    announce("graph + workspace growth on one handle")
    rng = np.random.default_rng(32)
    L, LONG = 3000, 200_000
    k, v = f16(rng, L + 1, G * D), f16(rng, L + 1, G * D)
    c = filled_cache(k[:L], v[:L], capacity=LONG)
    q, g = dev(f16(rng, H * D)), dev(f16(rng, H * D))
    kn, vn = dev(k[L]), dev(v[L])
    out = torch.empty(H * D, dtype=torch.float16, device="cuda")
    attn_step(c, 0, q, kn, vn, L, gate=g, out=out)  # sizes the workspace for L
    torch.cuda.synchronize()
    ref = out.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        attn_step(c, 0, q, kn, vn, L, gate=g, out=out)
    # growth refused under capture: the workspace (a long decode) and the cache
    refused = []
    g2 = torch.cuda.CUDAGraph()
    with warnings.catch_warnings(), torch.cuda.graph(g2):  # captures nothing: both refused
        warnings.simplefilter("ignore", UserWarning)
        for fn in (lambda: attn_decode(c, 0, q, LONG, out=torch.empty_like(out)),
                   lambda: attn_step(c, 0, q, kn, vn, 2 * LONG, out=torch.empty_like(out))):
            try:
                fn()
            except _lib.MiValueError as e:
                refused.append(str(e))
    del g2
    assert len(refused) == 2 and all("captur" in m for m in refused), refused
    # an eager long decode grows the workspace; the earlier graph still replays
    long_out = attn_decode(c, 0, q, LONG)
    torch.cuda.synchronize()
    assert torch.isfinite(long_out.float()).all()
    for r in range(3):
        out.fill_(7.0)
        graph.replay()
        attn_decode(c, 0, q, LONG, out=long_out)  # eager work on the grown workspace
        torch.cuda.synchronize()
        assert torch.equal(ref.view(torch.int16), out.view(torch.int16)), f"replay {r}"


def test_gate_extremes_decode_and_prefill():
    """Gate logits far in both tails (sigmoid -> 0 and -> 1, including values
    whose exponential overflows f32) and around 0, for the decode combine and
    the prefill epilogue, against the oracle's x / (1 + e^-g)."""
    announce("gate extremes")
    from moe_infer_amd import attn_prefill
    rng = np.random.default_rng(21)
    L = 300
    k, v = f16(rng, L, G * D), f16(rng, L, G * D)
    grid = np.array([-60000.0, -200.0, -90.0, -20.0, -3.0, -0.5, 0.0, 0.5, 3.0, 20.0, 90.0,
                     200.0, 60000.0], dtype=np.float32)
    q = f16(rng, H * D)
    g = np.resize(grid, H * D).astype(np.float16)
    c = filled_cache(k, v)
    out = attn_decode(c, 0, dev(q), L, gate=dev(g))
    assert_close(out, O.decode(q, k, v, L, gate=g), "decode gate extremes")
    n = 40
    qn, kn, vn = f16(rng, n, H, D), f16(rng, n, G * D), f16(rng, n, G * D)
    gn = np.resize(grid, n * H * D).reshape(n, H, D).astype(np.float16)
    c2 = Cache(num_layers=1, capacity=n)
    outp = attn_prefill(c2, 0, dev(qn), dev(kn), dev(vn), 0, gate=dev(gn))
    assert_close(outp, O.causal(qn, kn, vn, 0, gate=gn), "prefill gate extremes")


@pytest.mark.parametrize("Hq,Gk", [(32, 4), (8, 1)])
def test_other_head_counts(Hq, Gk):
    """Head counts other than 16 / 2 (eight query heads per KV head, the
    kernels' group size): decode, verify of 4 and 12 tokens (the grouped and
    wide forms) and prefill (its grid, and its split-K form after a long
    past) against the oracle."""
    from moe_infer_amd import attn_prefill
    announce(f"head counts H={Hq} G={Gk}")
    rng = np.random.default_rng(Hq + Gk)
    L = 3000
    k, v = f16(rng, L + 64, Gk * D), f16(rng, L + 64, Gk * D)
    c = Cache(num_layers=1, num_q_heads=Hq, num_kv_heads=Gk, capacity=L + 64)
    c.upload(0, k[:L], v[:L])
    c.set_pos(L)
    q1, g1 = f16(rng, Hq * D), f16(rng, Hq * D)
    out = attn_decode(c, 0, dev(q1), L, gate=dev(g1))
    assert_close(out, O.decode(q1, k, v, L, gate=g1, H=Hq, G=Gk), f"decode H={Hq}")
    for n in (4, 12):
        q, g = f16(rng, n, Hq, D), f16(rng, n, Hq, D)
        c.set_pos(L)
        out = attn_verify(c, 0, dev(q), dev(k[L:L + n]), dev(v[L:L + n]), L, gate=dev(g))
        ref = O.causal(q, k[:L + n], v[:L + n], L, gate=g, H=Hq, G=Gk)
        assert_close(out, ref, f"verify n={n} H={Hq}")
    for past, n in ((0, 300), (2500, 40)):  # the grid; the split-K form
        q = f16(rng, n, Hq, D)
        c.set_pos(past)
        out = attn_prefill(c, 0, dev(q), dev(k[past:past + n]), dev(v[past:past + n]), past)
        ref = O.causal(q, k[:past + n], v[:past + n], past, H=Hq, G=Gk)
        assert_close(out, ref, f"prefill past={past} n={n} H={Hq}")

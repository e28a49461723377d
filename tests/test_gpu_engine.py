"""The Engine surface (moe_infer_amd/engine.py) on the GPU: token-serial and
batched steps over the full-attention layers of a model config, the same
steps from projections (Q/K norm + RoPE fused in), the MTP draft head with
its verify / rollback / reset, position snapshots, cache transfer and
telemetry — each checked against the oracle's restatement of the reference
(attention: math_util.rs:264-392; norm + RoPE: math_util.rs:501-593; cache
semantics: cache.rs:84-128, mtp.rs:39-47)."""
import numpy as np
import pytest
import torch

from moe_infer_amd import Cache, Engine, record_engine_telemetry
from moe_infer_amd import engine as engine_mod
from oracle import oracle as O

from .conftest import f16
from .gpu_util import announce, assert_close, dev, host

pytestmark = pytest.mark.gpu
H, G, D = 16, 2, 256
# a reduced config of the reference's shape: 8 hidden layers, every 4th full
CONFIG = {"text_config": {"num_hidden_layers": 8, "num_attention_heads": H,
                          "num_key_value_heads": G, "head_dim": D,
                          "linear_num_value_heads": 32, "linear_num_key_heads": 16,
                          "rope_theta": 1e7, "partial_rotary_factor": 0.25,
                          "rms_norm_eps": 1e-6}}
FULL = [3, 7]


def test_config_maps_full_layers():
    c = Cache(CONFIG, capacity=256)
    assert c.full_layers == FULL
    with pytest.raises(ValueError):
        c.slot(2)
    e = Engine(c, config=CONFIG)
    assert e.rotary_dim == 64 and e.rope_theta == 1e7 and e.rms_norm_eps == 1e-6


def test_forward_token_serial():
    announce("engine forward")
    rng = np.random.default_rng(21)
    c = Cache(CONFIG, capacity=256)
    e = Engine(c, config=CONFIG)
    T = 40
    ks = {l: f16(rng, T, G * D) for l in FULL}
    vs = {l: f16(rng, T, G * D) for l in FULL}
    for t in range(T):
        qs = {l: f16(rng, H * D) for l in FULL}
        gs = {l: f16(rng, H * D) for l in FULL}
        outs = e.forward([(l, dev(qs[l]), dev(ks[l][t]), dev(vs[l][t]), dev(gs[l])) for l in FULL])
        assert e.engine_pos() == t + 1
        if t in (0, 17, T - 1):
            for l, out in zip(FULL, outs):
                assert_close(out, O.decode(qs[l], ks[l][:t + 1], vs[l][:t + 1], t + 1, gate=gs[l]),
                             f"forward t={t} layer={l}")


@pytest.mark.parametrize("n", [4, 16, 40])
def test_forward_batched_verify_and_prefill_routes(n):
    """n <= VERIFY_MAX_TOKENS goes to the split-K verify kernel, larger n to
    the prefill kernel; both equal the causal oracle after a serial prefix."""
    announce(f"engine forward_batched n={n}")
    assert (n <= engine_mod.VERIFY_MAX_TOKENS) == (n <= 16)
    rng = np.random.default_rng(n)
    c = Cache(CONFIG, capacity=256)
    e = Engine(c, config=CONFIG)
    P = 33
    kp = {l: f16(rng, P, G * D) for l in FULL}
    vp = {l: f16(rng, P, G * D) for l in FULL}
    for t in range(P):
        e.forward([(l, dev(f16(rng, H * D)), dev(kp[l][t]), dev(vp[l][t]), None) for l in FULL])
    q = {l: f16(rng, n, H, D) for l in FULL}
    k = {l: f16(rng, n, G * D) for l in FULL}
    v = {l: f16(rng, n, G * D) for l in FULL}
    g = {l: f16(rng, n, H, D) for l in FULL}
    outs = e.forward_batched([(l, dev(q[l]), dev(k[l]), dev(v[l]), dev(g[l])) for l in FULL])
    assert e.engine_pos() == P + n
    for l, out in zip(FULL, outs):
        ref = O.causal(q[l], np.concatenate([kp[l], k[l]]), np.concatenate([vp[l], v[l]]), P,
                       gate=g[l])
        assert_close(out, ref, f"forward_batched n={n} layer={l}")


def _proj_inputs(rng, n):
    q_proj = (rng.standard_normal((n, H, 2 * D)) * 2).astype(np.float32)
    k = (rng.standard_normal((n, G, D)) * 0.5).astype(np.float32)
    v = rng.standard_normal((n, G, D)).astype(np.float32)
    return q_proj, k, v


def _bf16(x):
    return torch.from_numpy(np.asarray(x, np.float32)).to(torch.bfloat16)


def _oracle_norm_rope(q_proj, k, qw, kw, pos0):
    qwb = qw.view(torch.int16).numpy().view(np.uint16)
    kwb = kw.view(torch.int16).numpy().view(np.uint16)
    n = q_proj.shape[0]
    qs, ks = [], []
    for t in range(n):
        qo, _ = O.q_head_norm_rope(q_proj[t], qwb, pos0 + t)
        ks.append(O.k_head_norm_rope(k[t], kwb, pos0 + t))
        qs.append(qo)
    return np.stack(qs), np.stack(ks)


def test_forward_proj_paths_match_oracle_chain():
    """forward_proj (fused step) token by token, then forward_batched_proj with
    n = 8 (verify route) and n = 24 (prefill route), against the oracle's
    norm + RoPE (rounded to f16 as the cache holds it) and its attention with
    the f32 gate."""
    announce("engine forward_proj / forward_batched_proj")
    rng = np.random.default_rng(77)
    c = Cache(CONFIG, capacity=256)
    e = Engine(c, config=CONFIG)
    qw = {l: _bf16(1 + 0.2 * rng.standard_normal(D)) for l in FULL}
    kw = {l: _bf16(1 + 0.2 * rng.standard_normal(D)) for l in FULL}
    krows = {l: [] for l in FULL}
    vrows = {l: [] for l in FULL}
    pos = 0
    for t in range(12):
        inp = {l: _proj_inputs(rng, 1) for l in FULL}
        outs = e.forward_proj([(l, torch.from_numpy(inp[l][0][0]).cuda(),
                                torch.from_numpy(inp[l][1][0]).cuda(),
                                torch.from_numpy(inp[l][2][0]).cuda(), qw[l].cuda(), kw[l].cuda())
                               for l in FULL])
        for l, out in zip(FULL, outs):
            qr, kr = _oracle_norm_rope(inp[l][0], inp[l][1], qw[l], kw[l], pos)
            krows[l].append(kr.reshape(1, G * D).astype(np.float16))
            vrows[l].append(inp[l][2].reshape(1, G * D).astype(np.float16))
            att = O.decode(qr[0].astype(np.float16), np.concatenate(krows[l]),
                           np.concatenate(vrows[l]), pos + 1)
            ref = O.sigmoid_gate(att.reshape(-1), inp[l][0][0, :, D:].reshape(-1))
            assert_close(out, ref, f"forward_proj t={t} layer={l}")
        pos += 1
    for n in (8, 24):
        inp = {l: _proj_inputs(rng, n) for l in FULL}
        outs = e.forward_batched_proj([(l, torch.from_numpy(inp[l][0]).cuda(),
                                        torch.from_numpy(inp[l][1]).cuda(),
                                        torch.from_numpy(inp[l][2]).cuda(), qw[l].cuda(),
                                        kw[l].cuda()) for l in FULL])
        assert e.engine_pos() == pos + n
        for l, out in zip(FULL, outs):
            qr, kr = _oracle_norm_rope(inp[l][0], inp[l][1], qw[l], kw[l], pos)
            krows[l].append(kr.reshape(n, G * D).astype(np.float16))
            vrows[l].append(inp[l][2].reshape(n, G * D).astype(np.float16))
            att = O.causal(qr.astype(np.float16), np.concatenate(krows[l]),
                           np.concatenate(vrows[l]), pos)
            ref = O.sigmoid_gate(att.reshape(-1), inp[l][0][:, :, D:].reshape(-1))
            assert_close(out, ref.reshape(n, H, D), f"forward_batched_proj n={n} layer={l}")
        pos += n


def test_mtp_head_verify_rollback_reset():
    """MTP state (mtp.rs:20-48): append-attend per draft step, K-token verify,
    rollback to an accepted prefix (rows untouched), reset to 0."""
    announce("engine mtp")
    rng = np.random.default_rng(5)
    c = Cache(CONFIG, capacity=256)
    e = Engine(c, mtp_capacity=256)
    K = [f16(rng, G * D) for _ in range(6)]
    V = [f16(rng, G * D) for _ in range(6)]
    for t in range(3):
        q, g = f16(rng, H * D), f16(rng, H * D)
        out = e.mtp_forward(dev(q), dev(K[t]), dev(V[t]), gate=dev(g))
        assert_close(out, O.decode(q, np.stack(K[:t + 1]), np.stack(V[:t + 1]), t + 1, gate=g),
                     f"mtp_forward {t}")
    assert e.mtp_pos == 3
    q4 = f16(rng, 3, H, D)
    out = e.mtp_verify(dev(q4), dev(np.stack(K[3:6])), dev(np.stack(V[3:6])))
    assert_close(out, O.causal(q4, np.stack(K), np.stack(V), 3), "mtp_verify")
    assert e.mtp_pos == 6
    e.mtp_rollback(4)
    assert e.mtp_pos == 4
    kd, vd = e.mtp_cache.download(0, rows=6)
    assert np.array_equal(kd.view(np.uint16), np.stack(K).view(np.uint16))  # rows untouched
    q, k5, v5 = f16(rng, H * D), f16(rng, G * D), f16(rng, G * D)
    out = e.mtp_forward(dev(q), dev(k5), dev(v5))
    assert_close(out, O.decode(q, np.stack(K[:4] + [k5]), np.stack(V[:4] + [v5]), 5),
                 "mtp after rollback")
    e.mtp_reset()
    assert e.mtp_pos == 0


def test_snapshot_restore_transfer_and_telemetry():
    announce("engine snapshot / transfer / telemetry")
    rng = np.random.default_rng(6)
    c = Cache(CONFIG, capacity=256)
    e = Engine(c, mtp_capacity=64)
    record_engine_telemetry(True)
    try:
        for t in range(5):
            e.forward([(l, dev(f16(rng, H * D)), dev(f16(rng, G * D)), dev(f16(rng, G * D)), None)
                       for l in FULL])
        snap = e.snapshot_state()
        assert (snap.pos, snap.mtp_pos) == (5, 0)
        e.forward([(l, dev(f16(rng, H * D)), dev(f16(rng, G * D)), dev(f16(rng, G * D)), None)
                   for l in FULL])
        e.mtp_forward(dev(f16(rng, H * D)), dev(f16(rng, G * D)), dev(f16(rng, G * D)))
        e.restore_snapshot(snap)
        assert e.engine_pos() == 5 and e.mtp_pos == 0 and c.len(3) == 5
        tel = e.telemetry()
        assert len(tel["engine.full_attention_ms"]) == 6
    finally:
        record_engine_telemetry(False)
    # download into a second cache and back: bit-identical rows and positions
    other = Cache(CONFIG, capacity=256)
    e.download_cache(other)
    assert other.pos == 5
    for l in FULL:
        a, b = c.download(l), other.download(l)
        assert np.array_equal(a[0].view(np.uint16), b[0].view(np.uint16))
        assert np.array_equal(a[1].view(np.uint16), b[1].view(np.uint16))
    other.set_pos(3)
    e.upload_cache(other)
    assert e.engine_pos() == 3
    assert not other.cpu_dirty

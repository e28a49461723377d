#!/usr/bin/env python3
"""Benchmark of the MI355X attention path at the BASELINE.json configs.

One JSON line on stdout.  The headline (`value`) is config C2: decode of one
token over a 32768-row f16 KV cache (16 query / 2 KV heads, head_dim 256,
sigmoid gate), reported as whole-call HBM GB/s.  One "step" runs that decode
over the 10 full-attention layers of Qwen3.6 (a distinct 64 MiB cache per
layer, so each launch reads K/V from HBM, not from the 256 MB last-level
cache).  Also reported: C4 causal prefill (4096 tokens, TFLOP/s), C5 K=4
verify at 65536 + rollback, C3 ragged 64-sequence decode, each with its
dominant kernel's duration from HIP events on its launch stream, and the CPU
baseline (the oracle's restatement of the reference CPU attention, one
thread, f32 inputs widened before timing) on bounded samples of C1 (ctx 512)
and of the C2 shape, with the host's CPU model.

Timing: launches are queued behind a GPU sleep so that the timed region
measures device execution, not Python enqueue cost; a barrier-free
single-process run (--gpus 1 only).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

H, G, D = 16, 2, 256
LAYERS = 10            # full-attention layers of Qwen3.6-35B-A3B
C2_CTX = 32768
C2_BYTES = 67_133_440  # K+V 67,108,864 + q, gate, out 3 x 8,192
C4_N = 4096
C4_FLOP = 4 * H * D * C4_N * (C4_N + 1) // 2  # QK^T + PV over causal pairs
C5_CTX, C5_K = 65536, 4
C5_BYTES = 134_324_224
C1_CTX = 512
C1_BYTES = 1_073_152  # K+V 1,048,576 + q, gate, out 3 x 8,192


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), or "unknown"."""
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--cpu-seconds", type=float, default=10.0,
                   help="bounded CPU-baseline sample length")
    p.add_argument("--only", default="", help="comma list of decode,prefill,verify,ragged,oproj,ceiling")
    p.add_argument("--copy-calib", action="store_true",
                   help="also run a plain 256 MiB device copy (reference for HBM counters)")
    return p.parse_args()


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build runs on one GPU; multi-GPU sharding is "
                          "designed (shard by KV head, then by context) but not built", "n_gpus": args.gpus}))
        sys.exit(2)

    import numpy as np
    import torch

    import moe_infer_amd as mi
    from moe_infer_amd import _lib

    torch.cuda.set_device(0)
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    only = set(filter(None, args.only.split(",")))
    hbm_peak, f16_peak = _lib.peaks()

    def randn(*shape, seed):
        gen.manual_seed(seed)
        return torch.randn(*shape, generator=gen, device=dev, dtype=torch.float32).half()

    # GPU sleep calibration: cycles per millisecond of torch.cuda._sleep
    def calib_sleep():
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(1000)
        torch.cuda.synchronize()
        s.record()
        torch.cuda._sleep(1_000_000)
        e.record()
        torch.cuda.synchronize()
        return 1_000_000 / max(s.elapsed_time(e), 1e-3)

    cyc_per_ms = calib_sleep()

    def timed(fn, steps, warmup, backlog_ms):
        """Runs fn() warmup + steps times; the timed steps are queued behind
        a GPU sleep of backlog_ms so the two events bracket device time only.
        A second pass of the same steps runs with the library's per-kernel
        events on (read afterwards with _lib.prof_read); those events add
        gaps between kernels, so they are kept out of the step timing."""
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(int(backlog_ms * cyc_per_ms))
        s.record()
        for _ in range(steps):
            fn()
        e.record()
        torch.cuda.synchronize()
        ms = s.elapsed_time(e) / steps  # ms per step
        _lib.prof_enable(True)
        torch.cuda._sleep(int(backlog_ms * cyc_per_ms))
        for _ in range(steps):
            fn()
        torch.cuda.synchronize()
        return ms

    print(f"[bench] start; sleep calib {cyc_per_ms:.0f} cycles/ms", file=sys.stderr, flush=True)
    rec = {}
    if args.copy_calib:  # a kernel of known traffic: reads and writes 256 MiB once each
        src = torch.empty(128 * 1024 * 1024, dtype=torch.float16, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    # ---------------------------------------------------------------- C2 decode
    if not only or "decode" in only:
        cache = mi.Cache(num_layers=LAYERS, capacity=C2_CTX)
        for layer in range(LAYERS):
            k = randn(C2_CTX, G * D, seed=200 + layer)
            v = randn(C2_CTX, G * D, seed=300 + layer)
            mi.kv_cache_append(cache, layer, k, v, 0)
            del k, v
        qs = [randn(H * D, seed=400 + i) for i in range(LAYERS)]
        gs = [randn(H * D, seed=500 + i) for i in range(LAYERS)]
        kn = [randn(G * D, seed=600 + i) for i in range(LAYERS)]
        vn = [randn(G * D, seed=700 + i) for i in range(LAYERS)]
        outs = [torch.empty(H * D, dtype=torch.float16, device=dev) for _ in range(LAYERS)]
        pos = C2_CTX - 1  # the step's own token is row 32767: it attends 32768 rows

        def decode_step():
            # the engine's per-layer attention step: append k, v at pos, attend
            # rows [0, pos], sigmoid gate (one fused launch pair per layer)
            for layer in range(LAYERS):
                mi.attn_step(cache, layer, qs[layer], kn[layer], vn[layer], pos, gate=gs[layer],
                             out=outs[layer])

        # the same step from the f32 projections (norm + RoPE + append + attend
        # + gate in the same two launches), as the engine would call it
        qp32 = [torch.randn(H * 2 * D, generator=gen.manual_seed(800 + i), device=dev)
                for i in range(LAYERS)]
        k32 = [torch.randn(G * D, generator=gen.manual_seed(900 + i), device=dev)
               for i in range(LAYERS)]
        v32 = [torch.randn(G * D, generator=gen.manual_seed(1000 + i), device=dev)
               for i in range(LAYERS)]
        qw = (1 + 0.1 * torch.randn(D, generator=gen.manual_seed(1100), device=dev)).bfloat16()
        kw = (1 + 0.1 * torch.randn(D, generator=gen.manual_seed(1101), device=dev)).bfloat16()

        def proj_step():
            for layer in range(LAYERS):
                mi.attn_step_proj(cache, layer, qp32[layer], k32[layer], v32[layer], qw, kw, pos,
                                  out=outs[layer])

        qo = [torch.empty(H, D, dtype=torch.float16, device=dev) for _ in range(LAYERS)]
        go = [torch.empty(H, D, dtype=torch.float16, device=dev) for _ in range(LAYERS)]

        def two_call_step():
            # the same step as two library calls: norm + RoPE + append, then
            # decode with the gate
            for layer in range(LAYERS):
                mi.qk_norm_rope_append(cache, layer, qp32[layer], k32[layer], v32[layer], qw, kw,
                                       pos, q_out=qo[layer], gate_out=go[layer])
                mi.attn_decode(cache, layer, qo[layer], C2_CTX, gate=go[layer], out=outs[layer])

        def attend_only():
            for layer in range(LAYERS):
                mi.attn_decode(cache, layer, qs[layer], C2_CTX, gate=gs[layer], out=outs[layer])

        ms = timed(decode_step, args.steps, args.warmup,
                   backlog_ms=args.steps * LAYERS * 0.25 + 20)
        split_us, n_split = _lib.prof_read("attn_split")
        comb_us, _ = _lib.prof_read("attn_combine")
        _lib.prof_enable(False)
        ms_attend = timed(attend_only, args.steps, args.warmup,
                          backlog_ms=args.steps * LAYERS * 0.25 + 20)
        _lib.prof_enable(False)
        ms_proj = timed(proj_step, args.steps, args.warmup,
                        backlog_ms=args.steps * LAYERS * 0.25 + 20)
        proj_split_us, _ = _lib.prof_read("attn_split")
        proj_comb_us, _ = _lib.prof_read("attn_combine")
        _lib.prof_enable(False)
        ms_two = timed(two_call_step, args.steps, args.warmup,
                       backlog_ms=args.steps * LAYERS * 0.35 + 20)
        rope_us, _ = _lib.prof_read("qk_norm_rope")
        _lib.prof_enable(False)
        # The same 10-layer step captured once as a HIP graph and replayed:
        # the 20 launches leave the host path (arguments are fixed per capture,
        # as in a serving loop that re-captures per position bucket).  The
        # replay must reproduce the eager outputs bit for bit.
        decode_step()
        torch.cuda.synchronize()
        eager = [o.clone() for o in outs]
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            decode_step()
        graph.replay()
        torch.cuda.synchronize()
        graph_ok = all(torch.equal(a.view(torch.int16), b.view(torch.int16))
                       for a, b in zip(eager, outs))
        ms_graph = timed(graph.replay, args.steps, args.warmup,
                         backlog_ms=args.steps * LAYERS * 0.25 + 20)
        _lib.prof_enable(False)
        del graph
        # The step followed by the layer's o_proj (bf16 2048 x 4096 per layer,
        # 10 x 16 MiB of weights) as the engine issues them: mi_attn_step,
        # then mi_matvec_bf16 of its output.
        od = 2048
        wos = [(randn(od, H * D, seed=1400 + i).float() * 0.05).to(torch.bfloat16)
               for i in range(LAYERS)]
        ys = [torch.empty(od, dtype=torch.float32, device=dev) for _ in range(LAYERS)]

        def step_then_oproj():
            for layer in range(LAYERS):
                mi.attn_step(cache, layer, qs[layer], kn[layer], vn[layer], pos, gate=gs[layer],
                             out=outs[layer])
                mi.matvec_bf16(outs[layer], wos[layer], out=ys[layer])

        ms_sep = timed(step_then_oproj, args.steps, args.warmup,
                       backlog_ms=args.steps * LAYERS * 0.3 + 20)
        sep_mv_us, _ = _lib.prof_read("matvec_bf16")
        _lib.prof_enable(False)
        del wos
        oproj_rec = {"us_per_layer": ms_sep * 1000 / LAYERS, "matvec_kernel_us": sep_mv_us,
                     "shape": [od, H * D],
                     "bytes_per_layer": C2_BYTES + od * H * D * 2 + od * 4}
        print(f"[bench] decode step + o_proj {ms_sep * 100:.2f} us/layer "
              f"(matvec kernel {sep_mv_us:.2f})", file=sys.stderr, flush=True)
        us_layer = ms * 1000 / LAYERS
        rec["decode"] = {
            "proj_step_us_per_layer": ms_proj * 1000 / LAYERS,
            "proj_split_kernel_us": proj_split_us, "proj_combine_kernel_us": proj_comb_us,
            "two_call_step_us_per_layer": ms_two * 1000 / LAYERS, "qk_norm_rope_kernel_us": rope_us,
            "us_per_layer": us_layer, "gbps": C2_BYTES / (us_layer * 1e3),
            "attend_only_us_per_layer": ms_attend * 1000 / LAYERS,
            "split_kernel_us": split_us, "combine_kernel_us": comb_us, "launches": n_split,
            "bytes_per_layer": C2_BYTES, "ms_per_step": ms,
            "graph_step_us_per_layer": ms_graph * 1000 / LAYERS,
            "graph_gbps": C2_BYTES / (ms_graph * 1e6 / LAYERS), "graph_matches_eager": graph_ok,
            "with_oproj": oproj_rec,
        }
        # Attend-only calls at other context lengths (the split plan depends on
        # the length), over 4 layers of 50000 rows (more than the last-level cache).
        del cache
        sweep_lens = (8193, 32769, 50000)
        scache = mi.Cache(num_layers=4, capacity=max(sweep_lens))
        for layer in range(4):
            k = randn(max(sweep_lens), G * D, seed=1200 + layer)
            v = randn(max(sweep_lens), G * D, seed=1300 + layer)
            mi.kv_cache_append(scache, layer, k, v, 0)
            del k, v
        sweep = {}
        for sl in sweep_lens:
            def attend_len(sl=sl):
                for layer in range(4):
                    mi.attn_decode(scache, layer, qs[layer], sl, gate=gs[layer], out=outs[layer])
            ms_sl = timed(attend_len, args.steps, args.warmup, backlog_ms=args.steps * 4 * 0.3 + 20)
            _lib.prof_enable(False)
            sweep[str(sl)] = {"us_per_call": ms_sl * 1000 / 4,
                              "gbps": (sl * G * D * 4 + 3 * H * D * 2) / (ms_sl * 1e6 / 4)}
        rec["decode"]["attend_by_ctx"] = sweep
        del scache
        print(f"[bench] decode step {us_layer:.2f} us/layer (attend only "
              f"{ms_attend * 100:.2f}, from projections {ms_proj * 100:.2f}: split "
              f"{proj_split_us:.2f} combine {proj_comb_us:.2f}; two calls {ms_two * 100:.2f}, "
              f"rope kernel {rope_us:.2f}) split {split_us:.2f} us combine {comb_us:.2f} us; "
              f"graph replay {ms_graph * 100:.2f} us/layer (matches eager: {graph_ok}); "
              + ", ".join(f"ctx {k_} {v_['us_per_call']:.2f} us" for k_, v_ in sweep.items()),
              file=sys.stderr, flush=True)

    # --------------------------------------------------------------- C4 prefill
    if not only or "prefill" in only:
        cache = mi.Cache(num_layers=1, capacity=C4_N)
        q = randn(C4_N, H, D, seed=41)
        k = randn(C4_N, G * D, seed=42)
        v = randn(C4_N, G * D, seed=43)
        out = torch.empty_like(q)

        def prefill_step():
            mi.attn_prefill(cache, 0, q, k, v, 0, out=out)

        psteps = max(args.steps, 10)
        ms = timed(prefill_step, psteps, args.warmup, backlog_ms=30)
        pk_us, _ = _lib.prof_read("attn_prefill")
        ap_us = _lib.prof_read("kv_pack")[0]
        _lib.prof_enable(False)
        # the same prefill with the sigmoid output gate (as the engine calls it)
        gate = randn(C4_N, H, D, seed=44)
        timed(lambda: mi.attn_prefill(cache, 0, q, k, v, 0, gate=gate, out=out), psteps,
              args.warmup, backlog_ms=30)
        pkg_us, _ = _lib.prof_read("attn_prefill")
        _lib.prof_enable(False)
        del gate
        rec["prefill"] = {
            "ms_per_step": ms, "kernel_us": pk_us, "append_us": ap_us,
            "tflops_kernel": C4_FLOP / (pk_us * 1e6), "tflops_step": C4_FLOP / (ms * 1e9),
            "flop": C4_FLOP, "kernel_us_gated": pkg_us,
        }
        print(f"[bench] prefill {ms * 1000:.1f} us/step kernel {pk_us:.1f} us "
              f"= {C4_FLOP / (pk_us * 1e6):.1f} TFLOP/s (gated kernel {pkg_us:.1f} us)",
              file=sys.stderr, flush=True)
        del cache

    # ---------------------------------------------------------------- C5 verify
    if not only or "verify" in only:
        nl = 4  # 4 x 128 MiB of K/V: more than the last-level cache
        cache = mi.Cache(num_layers=nl, capacity=C5_CTX + 16)
        for layer in range(nl):
            mi.kv_cache_append(cache, layer, randn(C5_CTX, G * D, seed=600 + layer),
                               randn(C5_CTX, G * D, seed=700 + layer), 0)
        q = randn(C5_K, H, D, seed=51)
        k = randn(C5_K, G * D, seed=52)
        v = randn(C5_K, G * D, seed=53)
        g = randn(C5_K, H, D, seed=54)
        out = torch.empty_like(q)

        def verify_step():
            for layer in range(nl):
                mi.attn_verify(cache, layer, q, k, v, C5_CTX, gate=g, out=out)
            cache.set_pos(C5_CTX + 2)  # accept 2 drafts, roll back the rest

        ms = timed(verify_step, args.steps, args.warmup, backlog_ms=args.steps * nl * 0.3 + 20)
        split_us, _ = _lib.prof_read("attn_split")
        _lib.prof_enable(False)
        us_call = ms * 1000 / nl
        rec["verify"] = {"us_per_layer": us_call, "gbps": C5_BYTES / (us_call * 1e3),
                         "split_kernel_us": split_us, "bytes": C5_BYTES}
        print(f"[bench] verify {us_call:.2f} us/layer", file=sys.stderr, flush=True)
        # The same call with 16 draft tokens: the wide verify (one split pass
        # reading each K/V tile once for all 16 tokens), and for comparison
        # the same tokens as four 4-token groups (MI_ATTN_VERIFY_WIDE=0).
        q16, k16 = randn(16, H, D, seed=55), randn(16, G * D, seed=56)
        v16, g16 = randn(16, G * D, seed=57), randn(16, H, D, seed=58)
        out16 = torch.empty_like(q16)

        def verify16():
            for layer in range(nl):
                mi.attn_verify(cache, layer, q16, k16, v16, C5_CTX, gate=g16, out=out16)
            cache.set_pos(C5_CTX + 2)

        ms16 = timed(verify16, args.steps, args.warmup, backlog_ms=args.steps * nl * 0.4 + 20)
        _lib.prof_enable(False)
        os.environ["MI_ATTN_VERIFY_WIDE"] = "0"
        try:
            ms16g = timed(verify16, args.steps, args.warmup,
                          backlog_ms=args.steps * nl * 1.2 + 20)
        finally:
            del os.environ["MI_ATTN_VERIFY_WIDE"]
        _lib.prof_enable(False)
        rec["verify"]["k16_us_per_layer"] = ms16 * 1000 / nl
        rec["verify"]["k16_grouped_us_per_layer"] = ms16g * 1000 / nl
        print(f"[bench] verify K=16 {ms16 * 1000 / nl:.2f} us/layer (as 4-token groups "
              f"{ms16g * 1000 / nl:.2f})", file=sys.stderr, flush=True)
        # Chunked prefill after a long past: 128 new tokens at 65536 rows,
        # the split-K form (default) against the prefill grid
        # (MI_ATTN_PREFILL_SPLIT=0).
        q128 = randn(128, H, D, seed=59)
        out128 = torch.empty_like(q128)

        def prefill_after_past():
            for layer in range(nl):
                cache.set_pos(C5_CTX + 16)
                mi.attn_prefill(cache, layer, q128, None, None, C5_CTX - 128,
                                out=out128)

        msp = timed(prefill_after_past, args.steps, args.warmup,
                    backlog_ms=args.steps * nl * 0.4 + 20)
        _lib.prof_enable(False)
        os.environ["MI_ATTN_PREFILL_SPLIT"] = "0"
        try:
            mspu = timed(prefill_after_past, max(2, args.steps // 4), 1,
                         backlog_ms=args.steps * nl * 2.0 + 20)
        finally:
            del os.environ["MI_ATTN_PREFILL_SPLIT"]
        _lib.prof_enable(False)
        rec["verify"]["prefill128_after_65408_us_per_layer"] = msp * 1000 / nl
        rec["verify"]["prefill128_after_65408_unsplit_us_per_layer"] = mspu * 1000 / nl
        print(f"[bench] prefill of 128 tokens after 65408 rows {msp * 1000 / nl:.1f} us/layer "
              f"(prefill grid {mspu * 1000 / nl:.1f})", file=sys.stderr, flush=True)
        del cache

    # ---------------------------------------------------------------- C3 ragged
    if not only or "ragged" in only:
        rng = np.random.default_rng(3)
        lengths = rng.integers(1024, 32769, size=64).astype(np.int32)
        offsets = np.zeros(64, np.int32)
        offsets[1:] = np.cumsum((lengths + 31) // 32 * 32)[:-1]
        rows = int(offsets[-1] + (lengths[-1] + 31) // 32 * 32)
        k, vb = mi.kv_pack(randn(rows, G * D, seed=31), randn(rows, G * D, seed=32), G)
        q = randn(64, H, D, seed=33)
        g = randn(64, H, D, seed=34)
        out = torch.empty_like(q)
        off_t = torch.from_numpy(offsets).to(dev)
        len_t = torch.from_numpy(lengths).to(dev)
        ws = mi.ragged_workspace(64, 32768, device=dev)
        mi.attn_decode_ragged(k, vb, off_t, len_t, q, 32768, gate=g, out=out, workspace=ws)

        def ragged_step():
            mi.attn_decode_ragged(k, vb, off_t, len_t, q, 32768, gate=g, out=out, workspace=ws,
                                  validate=False)

        ms = timed(ragged_step, args.steps, args.warmup, backlog_ms=20)
        split_us, _ = _lib.prof_read("attn_split")
        _lib.prof_enable(False)
        rbytes = 2048 * int(lengths.sum()) + 64 * 24576
        rec["ragged"] = {"us_per_step": ms * 1000, "gbps": rbytes / (ms * 1e6),
                         "split_kernel_us": split_us, "bytes": rbytes,
                         "sum_len": int(lengths.sum())}
        print(f"[bench] ragged {ms * 1000:.1f} us", file=sys.stderr, flush=True)
        del k, vb  # k holds the packed K blocks

    # ------------------------------------------------- o_proj matvec (bf16, q4)
    # out[2048] = W[2048, 4096] x[4096] after the gate; enough distinct weight
    # matrices that the set exceeds the 256 MiB last-level cache, as in a
    # model step where the layer's weights arrive cold.
    if not only or "oproj" in only:
        od, idim, gsz = 2048, H * D, 64
        nb, nq = 40, 96
        xs = randn(idim, seed=41)
        wb = [randn(od, idim, seed=900 + i).to(torch.bfloat16) for i in range(nb)]
        wq = [torch.randint(-2**31, 2**31 - 1, (od, idim // 8), dtype=torch.int32, device=dev)
              for _ in range(nq)]
        sq = torch.full((od, idim // gsz), 0.01, dtype=torch.bfloat16, device=dev)
        bq = torch.full((od, idim // gsz), -0.07, dtype=torch.bfloat16, device=dev)
        ob = torch.empty(od, dtype=torch.float32, device=dev)

        def bf16_step():
            for w in wb:
                mi.matvec_bf16(xs, w, out=ob)

        def q4_step():
            for w in wq:
                mi.matvec_q4(xs, w, sq, bq, group_size=gsz, out=ob)

        ms_b = timed(bf16_step, args.steps, args.warmup, backlog_ms=nb * 0.05 * args.steps + 20)
        kb_us, _ = _lib.prof_read("matvec_bf16")
        _lib.prof_enable(False)
        ms_q = timed(q4_step, args.steps, args.warmup, backlog_ms=nq * 0.02 * args.steps + 20)
        kq_us, _ = _lib.prof_read("matvec_q4")
        _lib.prof_enable(False)
        bytes_b = od * idim * 2 + idim * 2 + od * 4
        bytes_q = od * idim // 2 + 2 * od * (idim // gsz) * 2 + idim * 2 + od * 4
        rec["oproj"] = {"bf16_us": ms_b * 1000 / nb, "bf16_kernel_us": kb_us,
                        "bf16_gbps": bytes_b / (ms_b * 1e6 / nb), "bf16_bytes": bytes_b,
                        "q4_us": ms_q * 1000 / nq, "q4_kernel_us": kq_us,
                        "q4_gbps": bytes_q / (ms_q * 1e6 / nq), "q4_bytes": bytes_q,
                        "shape": [od, idim], "group_size": gsz}
        print(f"[bench] oproj bf16 {ms_b * 1000 / nb:.2f} us, q4 {ms_q * 1000 / nq:.2f} us",
              file=sys.stderr, flush=True)
        del wb, wq

    # ------------------------------------------------------------- MFMA ceiling
    # What the MFMA units reach on this part with nothing else in the loop:
    # one wave per SIMD on every CU, back-to-back v_mfma_f32_32x32x16_f16,
    # random N(0,1) operands and then zero operands (the data's share of the
    # power).  The prefill's fraction of nominal peak is read against this.
    if not only or "ceiling" in only:
        import ctypes as C
        wgs, iters = 256, 2048
        ops = randn(256 * 12 * 8, seed=51)
        cout = torch.empty(wgs * 256, dtype=torch.float32, device=dev)
        clk = torch.zeros(2 * wgs, dtype=torch.int64, device=dev)
        stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
        flop = wgs * 4 * iters * 8 * 32768
        ceil = {"workgroups": wgs, "waves_per_simd": 1, "mfma": "v_mfma_f32_32x32x16_f16",
                "flop_per_launch": flop}
        for name, o in (("random", ops), ("zero", torch.zeros_like(ops))):
            def launch():
                _lib.check(_lib.lib().mi_bench_mfma_ceiling(
                    C.c_void_p(o.data_ptr()), iters, wgs, C.c_void_p(cout.data_ptr()),
                    C.c_void_p(clk.data_ptr()), stream))
            for _ in range(5):
                launch()
            torch.cuda.synchronize()
            _lib.prof_enable(True)
            for _ in range(10):
                launch()
            torch.cuda.synchronize()
            us, _ = _lib.prof_read("mfma_ceiling")
            _lib.prof_enable(False)
            c = clk.cpu().numpy().reshape(wgs, 2).astype(np.float64)
            mhz = float(np.median(c[:, 0] / c[:, 1] * 100.0))
            tf = flop / (us * 1e-6) / 1e12
            ceil[name] = {"kernel_us": us, "tflops": tf, "frac_of_peak": tf / f16_peak,
                          "clock_mhz": mhz,
                          # clocks per MFMA per SIMD: 32 is full issue
                          "clk_per_mfma": float(np.median(c[:, 0])) / (iters * 8)}
        rec["mfma_ceiling"] = ceil
        print(f"[bench] mfma ceiling random {ceil['random']['tflops']:.0f} TFLOP/s "
              f"({ceil['random']['frac_of_peak']:.3f} of peak, {ceil['random']['clock_mhz']:.0f} MHz, "
              f"{ceil['random']['clk_per_mfma']:.1f} clk/MFMA); zero operands "
              f"{ceil['zero']['tflops']:.0f} TFLOP/s ({ceil['zero']['clock_mhz']:.0f} MHz)",
              file=sys.stderr, flush=True)

    # -------------------------------------------------------------- CPU baseline
    # The reference's CPU attention (src/math_util.rs:264-269, 323-383, one
    # thread as cpu.rs:149-163 runs it) on f32 inputs widened once outside
    # the timed loop, with the scores scratch allocated once: C1 (ctx 512)
    # and C2's shape (ctx 32768), each on a bounded sample.
    cpu = None
    if (not only or "decode" in only) and args.cpu_seconds > 0:
        from oracle import oracle as O
        rng = np.random.default_rng(2)
        qh = rng.standard_normal(H * D, dtype=np.float32).astype(np.float16)
        kh = rng.standard_normal((C2_CTX, G * D), dtype=np.float32).astype(np.float16)
        vh = rng.standard_normal((C2_CTX, G * D), dtype=np.float32).astype(np.float16)
        gh = rng.standard_normal(H * D, dtype=np.float32).astype(np.float16)
        base2 = O.DecodeBaseline(qh, kh, vh, gh)
        base1 = O.DecodeBaseline(qh, kh[:C1_CTX], vh[:C1_CTX], gh)

        def time_cpu(base, ctx, seconds):
            base.run(ctx)  # warm the caches and the library
            t0, runs = time.perf_counter(), 0
            while True:
                base.run(ctx)
                runs += 1
                el = time.perf_counter() - t0
                if el >= seconds:
                    return el / runs * 1e6, runs, el

        us1, runs1, el1 = time_cpu(base1, C1_CTX, args.cpu_seconds * 0.3)
        us2, runs2, el2 = time_cpu(base2, C2_CTX, args.cpu_seconds)
        # A labelled variant, not the baseline: the same loops with the 16
        # query heads spread over the host threads this job may use (16 on
        # the GPU box, whatever os.cpu_count() reports there).
        omp_threads = max(1, min(16, os.cpu_count() or 1))

        class _Omp:
            def run(self, ctx):
                base2.run_omp(ctx, omp_threads)

        us3, runs3, el3 = time_cpu(_Omp(), C2_CTX, args.cpu_seconds * 0.3)
        cpu = {"value": C2_BYTES / (us2 * 1e3), "unit": "GB/s", "cores": 1, "kind": "port",
               "us_per_layer": us2, "c1_us_per_layer": us1,
               "c1_gbps": C1_BYTES / (us1 * 1e3),
               "cpu_model": cpu_model(), "host_nproc": os.cpu_count(), "threads_used": 1,
               "build": O.build_flags(),
               "sample": f"C2 shape: {runs2} single-thread decodes (ctx 32768, gated) in "
                         f"{el2:.1f} s; C1: {runs1} decodes (ctx 512) in {el1:.1f} s; the C "
                         f"restatement of src/math_util.rs:264-269, 323-383 on f32 inputs "
                         f"widened once before timing, scores scratch preallocated",
               "omp_over_heads": {
                   "value": C2_BYTES / (us3 * 1e3), "unit": "GB/s", "threads": omp_threads,
                   "us_per_layer": us3,
                   "sample": f"C2 shape: {runs3} decodes in {el3:.1f} s, the same per-head "
                             f"loops with the query heads over {omp_threads} OpenMP threads "
                             f"(a labelled variant; the reference runs attention on one "
                             f"thread)"}}

    d = rec.get("decode")
    p = rec.get("prefill")
    line = {
        "metric": "decode attn µs/layer + HBM GB/s @ctx 32K; prefill TFLOP/s @4K tokens",
        "value": round(d["gbps"], 2) if d else None,
        "unit": "GB/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(d["ms_per_step"], 4) if d else None,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16", "data": "synthetic (seeded N(0,1) f16 q/K/V/gate)",
        "config": {"workload": "C2: GQA decode step (append the token's k/v, attend 32768 "
                               "rows, sigmoid gate), 16q/2kv heads, head_dim 256, f16 KV; "
                               "step = 10 full-attention layers",
                   "batch": 1, "ctx": C2_CTX, "layers_per_step": LAYERS},
    }
    # HBM bytes per launch measured by rocprofv3 counters (FETCH_SIZE + WRITE_SIZE,
    # scaled by a plain copy of known size) for the same command; see
    # profiles/attn_kernels_bench.md.  Null when the file is absent.
    traffic = {}
    tpath = ROOT / "profiles" / "traffic.json"
    if tpath.exists():
        traffic = json.loads(tpath.read_text())

    def traffic_of(key):
        e = traffic.get(key)
        return None if e is None else e["read_bytes"] + e["write_bytes"]

    # The traffic figures are not measured in this run: they come from the
    # committed counter runs, at the commit recorded in the file.
    traffic_src = ("profiles/traffic.json@" + str(traffic.get("commit", "unknown"))
                   + " (rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE; copy-scaled; not this run)"
                   if traffic else None)

    if d:
        line["decode_us_per_layer"] = round(d["us_per_layer"], 3)
        ach = C2_BYTES / (d["split_kernel_us"] * 1e3)
        line["roofline"] = {"bound": "hbm", "kernel": "attn_split_kernel (decode, C2)",
                            "achieved": round(ach, 1), "peak": hbm_peak, "unit": "GB/s",
                            "frac": round(ach / hbm_peak, 4),
                            "traffic": traffic_of("decode_split_c2"),
                            "traffic_source": traffic_src,
                            # the whole call (append + split + combine, launch gaps
                            # included): algorithmic bytes / step time per layer
                            "whole_call_achieved": round(d["gbps"], 1),
                            "whole_call_frac": round(d["gbps"] / hbm_peak, 4)}
        line["decode"] = {k2: (round(v2, 3) if isinstance(v2, float) else v2)
                          for k2, v2 in d.items()}
    if p:
        line["prefill_tflops"] = round(p["tflops_kernel"], 1)
        line["roofline_prefill"] = {"bound": "mfma", "kernel": "attn_prefill64_kernel (C4)",
                                    "achieved": round(p["tflops_kernel"], 1), "peak": f16_peak,
                                    "unit": "TFLOP/s",
                                    "frac": round(p["tflops_kernel"] / f16_peak, 4),
                                    "traffic": traffic_of("prefill_c4"),
                                    "traffic_source": traffic_src}
        line["prefill"] = {k2: (round(v2, 3) if isinstance(v2, float) else v2)
                           for k2, v2 in p.items()}
        mc = rec.get("mfma_ceiling")
        if mc:
            # the same kernel time against what MFMA alone reaches on this part
            line["roofline_prefill"]["frac_of_mfma_ceiling"] = round(
                p["tflops_kernel"] / mc["random"]["tflops"], 4)
    if "mfma_ceiling" in rec:
        line["mfma_ceiling"] = {k2: ({k3: round(v3, 3) for k3, v3 in v2.items()}
                                     if isinstance(v2, dict) else v2)
                                for k2, v2 in rec["mfma_ceiling"].items()}
    vr = rec.get("verify")
    if vr:
        ach = C5_BYTES / (vr["split_kernel_us"] * 1e3)
        line["roofline_verify"] = {"bound": "hbm", "kernel": "attn_split_kernel (verify, C5)",
                                   "achieved": round(ach, 1), "peak": hbm_peak, "unit": "GB/s",
                                   "frac": round(ach / hbm_peak, 4),
                                   "traffic": traffic_of("verify_split_c5"),
                            "traffic_source": traffic_src,
                                   "whole_call_achieved": round(vr["gbps"], 1),
                                   "whole_call_frac": round(vr["gbps"] / hbm_peak, 4)}
    for key in ("verify", "ragged", "oproj"):
        if key in rec:
            line[key] = {k2: (round(v2, 3) if isinstance(v2, float) else v2)
                         for k2, v2 in rec[key].items()}
    o = rec.get("oproj")
    if o:
        ach = o["bf16_bytes"] / (o["bf16_kernel_us"] * 1e3)
        line["roofline_oproj"] = {"bound": "hbm", "kernel": "matvec_bf16_kernel (o_proj 2048x4096)",
                                  "achieved": round(ach, 1), "peak": hbm_peak, "unit": "GB/s",
                                  "frac": round(ach / hbm_peak, 4),
                                  "traffic": traffic_of("oproj_bf16"),
                                    "traffic_source": traffic_src}
    line["cpu_baseline"] = cpu
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

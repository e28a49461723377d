"""Ragged batched decode and the KV-cache state operations on the GPU:
append / upload / download bit-exactness, position-only rollback, reset,
doubling growth, copy_from and save/load (src/cache.rs semantics, modelled
by oracle.CacheModel)."""
import json
import numpy as np
import pytest
import torch

from moe_infer_amd import Cache, attn_decode, attn_decode_ragged, kv_cache_append, kv_pack
from oracle import oracle as O

from .conftest import f16
from .gpu_util import announce, assert_close, dev, host

pytestmark = pytest.mark.gpu
H, G, D = 16, 2, 256


def ragged_buffers(rng, lengths):
    offsets, rows = [], 0
    for n in lengths:
        offsets.append(rows)
        rows += (n + 31) // 32 * 32  # sequences start on a 32-row block
    rows = max(rows, 32)
    k, v = f16(rng, rows, G * D), f16(rng, rows, G * D)
    return np.array(offsets, np.int32), k, v


@pytest.mark.parametrize("lengths", [[5, 0, 17, 1, 8, 9, 33, 300],
                                     [1024, 1, 2049, 255, 4096, 0, 777, 129],
                                     [60000, 3]])  # one sequence over every workgroup
def test_ragged_matches_oracle(lengths):
    announce(f"ragged {lengths}")
    rng = np.random.default_rng(sum(lengths))
    lengths = np.array(lengths, np.int32)
    offsets, k, v = ragged_buffers(rng, lengths)
    b = len(lengths)
    q, g = f16(rng, b, H, D), f16(rng, b, H, D)
    kb, vb = kv_pack(dev(k), dev(v), G)
    out = attn_decode_ragged(kb, vb, torch.from_numpy(offsets).cuda(),
                             torch.from_numpy(lengths).cuda(), dev(q), int(lengths.max()),
                             gate=dev(g))
    ref = O.decode_ragged(q, k, v, offsets, lengths, gate=g)
    assert_close(out, ref, f"ragged {list(lengths)}")
    o = host(out)
    assert np.all(o[lengths == 0] == 0)


def test_ragged_c3_shape():
    """64 sequences, lengths U[1024, 32768] (seed 3);
    8 sequences are checked against the oracle, all 64 against the GPU
    single-sequence decode of the same rows (ragged == independent decodes)."""
    announce("ragged C3 64 seqs")
    rng = np.random.default_rng(3)
    lengths = rng.integers(1024, 32769, size=64).astype(np.int32)
    offsets, k, v = ragged_buffers(rng, lengths)
    q = f16(rng, 64, H, D)
    kb, vb = kv_pack(dev(k), dev(v), G)
    out = host(attn_decode_ragged(kb, vb, torch.from_numpy(offsets).cuda(),
                                  torch.from_numpy(lengths).cuda(), dev(q), 32768))
    for s in range(0, 64, 8):
        a, n = offsets[s], lengths[s]
        assert_close(out[s], O.decode(q[s], k[a:a + n], v[a:a + n], n), f"C3 seq {s} (L={n})")
    c = Cache(num_layers=1, capacity=32768)
    for s in range(64):
        a, n = offsets[s], lengths[s]
        c.upload(0, k[a:a + n], v[a:a + n])
        dec = host(attn_decode(c, 0, dev(q[s]), int(n)))
        # different split-K chunking: equal up to f32 re-association
        assert_close(out[s], dec.reshape(H, D), f"C3 seq {s} vs decode", atol=5e-4)


def test_ragged_rejects_bad_tables():
    rng = np.random.default_rng(0)
    k, v = f16(rng, 64, G * D), f16(rng, 64, G * D)
    kb, vb = kv_pack(dev(k), dev(v), G)
    q = dev(f16(rng, 2, H, D))
    for off, ln in (([0, 8], [4, 4]), ([0, 32], [4, 100]), ([0, 32], [4, -1]), ([0, 32], [4, 33])):
        with pytest.raises(ValueError):
            attn_decode_ragged(kb, vb, torch.tensor(off, dtype=torch.int32).cuda(),
                               torch.tensor(ln, dtype=torch.int32).cuda(), q, 64)


@pytest.mark.parametrize("b", [600, 256, 200])
def test_ragged_many_sequences_flat_split(b):
    """Many sequences, lengths 0..300 with exact multiples of 32 among them:
    every output equals the oracle, zero-length sequences are zero.  600 runs
    the plan kernel's scan over three 256-sequence blocks; 256 and 200 the
    split launch's own scan (full and partial last 64-lane step)."""
    announce(f"ragged {b} seqs")
    rng = np.random.default_rng(b)
    lengths = rng.integers(0, 301, size=b).astype(np.int32)
    lengths[::7] = 0
    lengths[3::11] = 64
    lengths[5::13] = 32
    offsets, k, v = ragged_buffers(rng, lengths)
    b = len(lengths)
    q, g = f16(rng, b, H, D), f16(rng, b, H, D)
    kb, vb = kv_pack(dev(k), dev(v), G)
    out = attn_decode_ragged(kb, vb, torch.from_numpy(offsets).cuda(),
                             torch.from_numpy(lengths).cuda(), dev(q), int(lengths.max()),
                             gate=dev(g))
    ref = O.decode_ragged(q, k, v, offsets, lengths, gate=g)
    assert_close(out, ref, f"ragged {b} seqs")
    assert np.all(host(out)[lengths == 0] == 0)


def test_ragged_invalid_rows_report_nan_on_device():
    """With host validation off, sequences whose descriptor is invalid
    (unaligned offset, length past max_len, negative length) come out NaN;
    the others are unaffected."""
    announce("ragged invalid descriptors (device)")
    rng = np.random.default_rng(9)
    lengths = np.array([40, 50, 60, 70, 80], np.int32)
    offsets, k, v = ragged_buffers(rng, lengths)
    q = f16(rng, 5, H, D)
    kb, vb = kv_pack(dev(k), dev(v), G)
    bad_off = offsets.copy()
    bad_len = lengths.copy()
    bad_off[1] += 8         # not on a 32-row block
    bad_len[3] = 1000       # past max_len
    bad_len[4] = -2
    out = host(attn_decode_ragged(kb, vb, torch.from_numpy(bad_off).cuda(),
                                  torch.from_numpy(bad_len).cuda(), dev(q), 100,
                                  validate=False))
    assert np.all(np.isnan(out[[1, 3, 4]]))
    for s in (0, 2):
        a, n = offsets[s], lengths[s]
        assert_close(out[s], O.decode(q[s], k[a:a + n], v[a:a + n], n), f"valid seq {s}")


def test_pack_layout():
    """Rows land where mi_attn.h documents: K at
    (((b*G + h)*2 + u)*(D/8) + i/8)*128 + j*8 + i%8 with r = 32b + w,
    u = (w/4)%2, j = 4*(w/8) + w%4; V at ((r/8)*G + h)*D*8 + i*8 + r%8."""
    rng = np.random.default_rng(11)
    n = 45
    k, v = f16(rng, n, G * D), f16(rng, n, G * D)
    kb, vb = (host(t) for t in kv_pack(dev(k), dev(v), G))
    kb = kb.reshape(-1, G, 2, D // 8, 16, 8)
    vb = vb.reshape(-1, G, D, 8)
    for r in range(n):
        b, w = divmod(r, 32)
        u, j = (w // 4) % 2, 4 * (w // 8) + w % 4
        for h in range(G):
            assert np.array_equal(kb[b, h, u, :, j, :].reshape(D).view(np.uint16),
                                  k[r, h * D:(h + 1) * D].view(np.uint16))
            assert np.array_equal(vb[r // 8, h, :, r % 8].view(np.uint16),
                                  v[r, h * D:(h + 1) * D].view(np.uint16))


def test_append_download_bit_exact_and_rollback():
    announce("cache append/rollback")
    rng = np.random.default_rng(12)
    layers, cap = 3, 64
    c = Cache(num_layers=layers, capacity=cap)
    m = O.CacheModel(layers, G * D, c.capacity)
    pos = 0
    for step, n in enumerate([1, 3, 8, 13, 1, 40, 7]):
        for layer in range(layers):
            k, v = f16(rng, n, G * D), f16(rng, n, G * D)
            kv_cache_append(c, layer, dev(k), dev(v), pos)
            m.append(layer, k, v, pos)
            assert c.len(layer) == m.len[layer]
        pos += n
        if step == 3:  # roll back 5 rows: nothing is erased
            pos -= 5
            c.set_pos(pos)
            m.set_pos(pos)
    torch.cuda.synchronize()
    for layer in range(layers):
        kd, vd = c.download(layer, rows=c.capacity)
        mk, mv = m.k[layer][:c.capacity], m.v[layer][:c.capacity]
        assert np.array_equal(kd.view(np.uint16), mk.view(np.uint16))
        assert np.array_equal(vd.view(np.uint16), mv.view(np.uint16))
    c.reset()
    assert c.pos == 0 and all(c.len(i) == 0 for i in range(layers))
    kd, _ = c.download(0, rows=pos)
    assert np.array_equal(kd.view(np.uint16), m.k[0][:pos].view(np.uint16))  # reset erases nothing


@pytest.mark.parametrize("row0,n", [(37, 300), (64, 128), (5, 1000), (96, 130), (3, 127), (31, 129)])
def test_long_unaligned_append_keeps_neighbours(row0, n):
    """Appends of 128 rows or more take the destination-ordered K path, fewer
    the row-major one (n = 127): rows before row0 and from row0 + n on keep
    their contents, and the appended rows land, bit for bit."""
    announce(f"long append row0={row0} n={n}")
    rng = np.random.default_rng(row0 * 7 + n)
    c = Cache(num_layers=1, capacity=2048)
    cap = c.capacity
    base_k, base_v = f16(rng, cap, G * D), f16(rng, cap, G * D)
    c.upload(0, base_k, base_v)
    k, v = f16(rng, n, G * D), f16(rng, n, G * D)
    c.set_pos(row0)
    kv_cache_append(c, 0, dev(k), dev(v), row0)
    ek, ev = base_k.copy(), base_v.copy()
    ek[row0:row0 + n], ev[row0:row0 + n] = k, v
    kd, vd = c.download(0, rows=cap)
    assert np.array_equal(kd.view(np.uint16), ek.view(np.uint16))
    assert np.array_equal(vd.view(np.uint16), ev.view(np.uint16))


def test_upload_unaligned_rows_and_growth():
    rng = np.random.default_rng(13)
    c = Cache(num_layers=1, capacity=256)
    base_k, base_v = f16(rng, 256, G * D), f16(rng, 256, G * D)
    c.upload(0, base_k, base_v)
    k, v = f16(rng, 11, G * D), f16(rng, 11, G * D)
    c.upload(0, k, v, row0=5)  # partial V blocks on both ends
    ek, ev = base_k.copy(), base_v.copy()
    ek[5:16], ev[5:16] = k, v
    kd, vd = c.download(0, rows=256)
    assert np.array_equal(kd.view(np.uint16), ek.view(np.uint16))
    assert np.array_equal(vd.view(np.uint16), ev.view(np.uint16))
    c.set_pos(200)
    kx, vx = f16(rng, 100, G * D), f16(rng, 100, G * D)
    kv_cache_append(c, 0, dev(kx), dev(vx), 250)  # grows 256 -> 512, keeps every row
    assert c.capacity == 512 and c.len(0) == 350
    kd, vd = c.download(0, rows=350)
    assert np.array_equal(kd[:250].view(np.uint16), ek[:250].view(np.uint16))
    assert np.array_equal(vd[:250].view(np.uint16), ev[:250].view(np.uint16))
    assert np.array_equal(vd[250:].view(np.uint16), vx.view(np.uint16))


def test_copy_from_and_save_load(tmp_path):
    rng = np.random.default_rng(14)
    cfg = {"num_hidden_layers": 8, "num_attention_heads": 16, "num_key_value_heads": 2,
           "head_dim": 256, "linear_num_value_heads": 32, "linear_num_key_heads": 16}
    c = Cache(cfg, capacity=300)
    assert c.full_layers == [3, 7]
    with pytest.raises(ValueError):
        c.slot(2)
    for layer in c.full_layers:
        kv_cache_append(c, layer, dev(f16(rng, 77, G * D)), dev(f16(rng, 77, G * D)), 0)
    c.set_pos(70)
    c.set_len(7, 77)
    d = Cache(cfg, capacity=16)
    d.copy_from(c)
    assert d.pos == 70 and d.len(3) == 70 and d.len(7) == 77 and d.capacity == c.capacity
    bin_p, json_p = str(tmp_path / "c.bin"), str(tmp_path / "c.json")
    c.save(bin_p, json_p)
    e = Cache.load(bin_p, json_p, cfg)
    assert e.pos == 70 and e.len(3) == 70 and e.len(7) == 77
    for layer in c.full_layers:
        a, b, x = c.download(layer, rows=c.capacity), d.download(layer, rows=c.capacity), \
            e.download(layer, rows=c.capacity)
        for i in range(2):
            assert np.array_equal(a[i].view(np.uint16), b[i].view(np.uint16))
            assert np.array_equal(a[i].view(np.uint16), x[i].view(np.uint16))


def _write_reference_cache(bin_p, json_p, n_layers, full, rows, kv_dim, k, v, lens, pos):
    """A cache file in the reference's layout (cache.rs:133-177, 236-270):
    per layer in order either k_cache / v_cache float32 [rows, kv_dim] + len
    uint32, or the linear layer's conv_state / ssm_state float32; cache.pos
    last; native-endian; offsets in a JSON manifest."""
    tensors, off = {}, 0
    with open(bin_p, "wb") as f:
        def put(name, arr, shape, dtype):
            nonlocal off
            b = arr.tobytes()
            f.write(b)
            tensors[name] = {"offset": off, "size": len(b), "shape": shape, "dtype": dtype}
            off += len(b)
        for i in range(n_layers):
            if i in full:
                put(f"cache.layer_{i}.k_cache", k[i].astype(np.float32), [rows, kv_dim], "float32")
                put(f"cache.layer_{i}.v_cache", v[i].astype(np.float32), [rows, kv_dim], "float32")
                put(f"cache.layer_{i}.len", np.array([lens[i]], np.uint32), [], "uint32")
            else:
                put(f"cache.layer_{i}.conv_state", np.full((3, 8), 7.0, np.float32), [3, 8],
                    "float32")
                put(f"cache.layer_{i}.ssm_state", np.full(16, -3.0, np.float32), [16], "float32")
        put("cache.pos", np.array([pos], np.uint32), [], "uint32")
    with open(json_p, "w") as f:
        json.dump({"tensors": tensors}, f, indent=2)


def test_load_reference_float32_file(tmp_path):
    """A file in the reference's float32 layout, with the linear layers' state
    in between, loads into the f16 cache: rows are the f16 rounding of the f32
    values, len per layer and pos as stored; saving writes float16 with the
    same names, shapes and order, and loads back bit for bit."""
    rng = np.random.default_rng(15)
    cfg = {"num_hidden_layers": 8, "num_attention_heads": 16, "num_key_value_heads": 2,
           "head_dim": 256, "linear_num_value_heads": 32, "linear_num_key_heads": 16}
    rows, kv_dim, full = 256, G * D, [3, 7]
    k = {i: rng.standard_normal((rows, kv_dim)).astype(np.float32) for i in full}
    v = {i: rng.standard_normal((rows, kv_dim)).astype(np.float32) for i in full}
    lens = {3: 100, 7: 101}
    bin_p, json_p = str(tmp_path / "ref.bin"), str(tmp_path / "ref.json")
    _write_reference_cache(bin_p, json_p, 8, full, rows, kv_dim, k, v, lens, 100)
    c = Cache.load(bin_p, json_p, cfg)
    assert c.pos == 100 and c.len(3) == 100 and c.len(7) == 101
    for i in full:
        kd, vd = c.download(i, rows=rows)
        assert np.array_equal(kd.view(np.uint16), k[i].astype(np.float16).view(np.uint16))
        assert np.array_equal(vd.view(np.uint16), v[i].astype(np.float16).view(np.uint16))
    out_bin, out_json = str(tmp_path / "f16.bin"), str(tmp_path / "f16.json")
    c.save(out_bin, out_json)
    with open(out_json) as f:
        man = json.load(f)["tensors"]
    names = sorted(man, key=lambda n: man[n]["offset"])
    assert names == ["cache.layer_3.k_cache", "cache.layer_3.v_cache", "cache.layer_3.len",
                     "cache.layer_7.k_cache", "cache.layer_7.v_cache", "cache.layer_7.len",
                     "cache.pos"]
    assert man["cache.layer_3.k_cache"]["dtype"] == "float16"
    assert man["cache.layer_3.k_cache"]["shape"] == [c.capacity, kv_dim]
    e = Cache.load(out_bin, out_json, cfg)
    assert e.pos == 100 and e.len(7) == 101
    for i in full:
        a, b = c.download(i, rows=rows), e.download(i, rows=rows)
        assert np.array_equal(a[0].view(np.uint16), b[0].view(np.uint16))
        assert np.array_equal(a[1].view(np.uint16), b[1].view(np.uint16))


def test_growth_after_queued_appends_on_a_side_stream():
    """Appends queued on a non-blocking stream, then a step past the capacity
    (which regrows the cache) on the same stream without a host sync: the
    regrow waits for the queued appends, so every row survives the copy."""
    announce("growth after queued appends on a side stream")
    rng = np.random.default_rng(17)
    c = Cache(num_layers=1, capacity=256)
    T = 260
    ks, vs = f16(rng, T, G * D), f16(rng, T, G * D)
    kd_all, vd_all = dev(ks), dev(vs)
    q = dev(f16(rng, H * D))
    s = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        for t in range(T):
            out = attn_step_wrapper(c, q, kd_all[t], vd_all[t], t)
    s.synchronize()
    assert c.capacity >= T
    kd, vd = c.download(0, rows=T)
    assert np.array_equal(kd.view(np.uint16), ks.view(np.uint16))
    assert np.array_equal(vd.view(np.uint16), vs.view(np.uint16))
    assert_close(out, O.decode(host(q), ks, vs, T), "decode after growth on a side stream")


def attn_step_wrapper(c, q, k, v, t):
    from moe_infer_amd import attn_step
    return attn_step(c, 0, q, k, v, t)

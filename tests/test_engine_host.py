"""Host logic of Engine on the CPU (no kernel runs): the per-layer interrupt
poll of the forward methods, as the reference polls check_signal() before
each layer and returns MoEError::Metal("interrupted") without advancing the
position (src/engine/qwen35_moe/fused_exp2.rs:1017-1019,
src/python_bindings.rs:152)."""
import pytest

import moe_infer_amd.engine as E


class FakeCache:
    num_q_heads, num_kv_heads, head_dim = 16, 2, 256

    def __init__(self, pos):
        self.pos = pos
        self.gpu_dirty = False
        self.lens = {}

    def set_pos(self, p):
        self.pos = p

    def set_len(self, layer, n):
        self.lens[layer] = n


class FakeTensor:
    def __init__(self, numel):
        self._n = numel

    def numel(self):
        return self._n


def make_engine(pos):
    eng = E.Engine.__new__(E.Engine)  # no device cache: the attention calls are stubbed
    eng.cache = FakeCache(pos)
    eng.rotary_dim, eng.rope_theta, eng.rms_norm_eps = 64, 1e7, 1e-6
    eng._telemetry = {}
    return eng


@pytest.fixture
def calls(monkeypatch):
    log = []
    for name in ("attn_step", "attn_verify", "attn_prefill", "attn_step_proj"):
        monkeypatch.setattr(E.attention, name,
                            lambda cache, layer, *a, _n=name, **kw: log.append((_n, layer)) or _n)
    monkeypatch.setattr(E.attention, "qk_norm_rope_append",
                        lambda cache, layer, *a, **kw: (log.append(("rope", layer)), ("q", "g"))[1])
    return log


def polls_true_at(k):
    state = {"n": 0}

    def check():
        state["n"] += 1
        return state["n"] > k
    return check, state


@pytest.mark.parametrize("method", ["forward", "forward_batched", "forward_proj",
                                    "forward_batched_proj"])
def test_interrupt_before_a_layer_raises_and_keeps_pos(method, calls):
    eng = make_engine(pos=41)
    H, D = 16, 256
    if method == "forward":
        layers = [(l, None, None, None, None) for l in (3, 7, 11)]
    elif method == "forward_batched":
        layers = [(l, FakeTensor(4 * H * D), None, None, None) for l in (3, 7, 11)]
    else:
        layers = [(l, FakeTensor(4 * H * 2 * D), None, None, None, None) for l in (3, 7, 11)]
    check, state = polls_true_at(2)
    with pytest.raises(E.EngineInterrupted) as ei:
        getattr(eng, method)(layers, check_signal=check)
    assert isinstance(ei.value, RuntimeError) and "interrupted" in str(ei.value)
    assert eng.engine_pos() == 41, "an interrupted call does not advance the position"
    assert state["n"] == 3, "polled once per layer, before the layer"
    assert [c[1] for c in calls if c[0] != "rope"] == [3, 7]
    # the layers that ran (and appended rows) have their len put back to pos
    assert eng.cache.lens == {3: 41, 7: 41}


@pytest.mark.parametrize("method", ["forward", "forward_batched"])
def test_no_interrupt_runs_every_layer_and_advances(method, calls):
    eng = make_engine(pos=10)
    n = 1 if method == "forward" else 20
    layers = [(l, FakeTensor(n * 16 * 256), None, None, None) for l in range(4)]
    check, state = polls_true_at(100)
    outs = getattr(eng, method)(layers, check_signal=check)
    assert len(outs) == 4 and state["n"] == 4
    assert eng.engine_pos() == 10 + n
    if method == "forward_batched":  # n = 20 > the verify limit: the prefill kernel
        assert {c[0] for c in calls} == {"attn_prefill"}

"""The kernels' reads stay inside the cache allocation, checked on the CPU
by a model of their tile walks compiled against the launch-plan header the
kernels themselves use (moe_infer_amd/csrc/plan.h): the causal prefill's
global -> LDS tile copies (both kernel forms, the 64-query one over both of
its passes) over (past, n) in [0, 700)^2 and at long pasts,
the split-K decode / verify tile loads over lengths 1..5000 and long
contexts under several planning knobs, and the wide verify / split-K
prefill's tile copies (mi::wide_plan, mi::verify_wave64) over pasts up to
131071 and 1..1100 tokens.  The prefill walk without the
steady schedule's last-tile rule must find out-of-allocation copies (the
fault that rule fixed), so the model is shown to catch it."""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


@pytest.fixture(scope="module")
def model_output(tmp_path_factory):
    cxx = shutil.which("g++")
    if cxx is None:
        pytest.skip("g++ not available")
    exe = tmp_path_factory.mktemp("bounds") / "copy_bounds_model"
    subprocess.run([cxx, "-O2", "-std=c++17", f"-I{ROOT / 'moe_infer_amd' / 'csrc'}",
                    str(ROOT / "tests" / "copy_bounds_model.cc"), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True,
                         timeout=600).stdout
    res = {}
    for ln in out.splitlines():
        name, cases, bad = ln.split()
        res[name] = (int(cases), int(bad))
    return res


def test_prefill_tile_copies_stay_inside_the_allocation(model_output):
    cases, bad = model_output["prefill"]
    assert cases == 700 * 699 and bad == 0


def test_prefill64_tile_copies_stay_inside_the_allocation(model_output):
    cases, bad = model_output["prefill64"]
    assert cases == 700 * 699 and bad == 0


def test_prefill_model_catches_the_copy_past_the_last_tile(model_output):
    cases, bad = model_output["prefill_without_last_tile_rule"]
    assert bad > 0, "the model must flag the steady schedule's K(t+1) copy on the last tile"


def test_prefill_long_past_and_c4_sizes(model_output):
    cases, bad = model_output["prefill_long"]
    assert cases == 45 and bad == 0


def test_split_tiles_are_whole_and_inside_the_allocation(model_output):
    cases, bad = model_output["split"]
    assert cases > 0 and bad == 0


def test_wide_verify_tiles_stay_inside_the_allocation(model_output):
    """The wide verify / split-K prefill: every tile copy inside the cache,
    chunks whole tiles covering every row, each token's visible keys walked."""
    cases, bad = model_output["wide"]
    assert cases > 500 and bad == 0

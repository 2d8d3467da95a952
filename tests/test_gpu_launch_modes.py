"""Decode launch modes and the wait error path, each run in a child process
with its own environment (the decoder reads these knobs once per process).

* FMD_ATTN_SPIN_LIMIT=0: a wait of the single-launch attention that is not
  satisfied at its first poll gives up at once.  The launch must still drain,
  the call must fail with the spin-limit error instead of hanging, and the
  steps before the first failure must match a normal run.
* FMD_PROJ_CHAIN=1 (a layer's O, gate|up and down projections in one
  launch) and FMD_DECODE_LAYERS=1 (every layer in one launch) must give the
  default path's logits within the decode tolerance.
* FMD_GEMM_BLDS=0 and =2 (prefill GEMM weight fragments never / always
  staged through LDS; by default only 64-row tiles stage them) must give
  bit-identical prefill logits and K/V: every form feeds the same operands
  to the same MFMAs in the same order.
"""
import json
import os
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

from tests.gpu_util import TOL

pytestmark = pytest.mark.gpu

CHILD = Path(__file__).resolve().parent / "gpu_child.py"
KNOBS = ("FMD_ATTN_SPIN_LIMIT", "FMD_PROJ_CHAIN", "FMD_DECODE_LAYERS", "FMD_GEMM_BLDS")


def _run(tmp_path, env_extra, cfg="tiny", prec="int8", steps=6, timeout=150, mode="decode"):
    env = {k: v for k, v in os.environ.items() if k not in KNOBS}
    env.update(env_extra)
    tag = '_'.join(f'{k}{v}' for k, v in env_extra.items()) or 'base'
    out = tmp_path / f"{cfg}_{prec}_{mode}_{tag}.npz"
    print(f"[gpu] child {cfg} {prec} {mode} {env_extra}", flush=True)
    r = subprocess.run([sys.executable, str(CHILD), cfg, prec, str(steps), str(out), mode], env=env,
                       capture_output=True, text=True, timeout=timeout)
    assert r.returncode == 0, r.stderr[-3000:]
    info = json.loads(r.stdout.strip().splitlines()[-1])
    z = np.load(out)
    info["logits"], info["steps"] = z["logits"], z["steps"]
    if "cache" in z:
        info["cache"] = z["cache"]
    return info


def test_wait_error_path_drains_and_reports(tmp_path):
    base = _run(tmp_path, {})
    assert not base["errors"] and len(base["steps"]) == 6
    got = _run(tmp_path, {"FMD_ATTN_SPIN_LIMIT": "0"})
    for e in got["errors"]:
        assert "did not meet within the spin limit" in e, e
    assert got["len"] == base["len"]
    # a failed step still appends its (possibly wrong) K/V, so only the steps
    # before the first failure must reproduce the normal run
    ok = [int(s) for s in got["steps"]]
    first_err = next((s for s in range(6) if s not in ok), 6)
    for i, s in enumerate(ok):
        if s < first_err:
            d = np.max(np.abs(got["logits"][i] - base["logits"][s]))
            assert d < TOL["int8"], (s, d)
    if not got["errors"]:
        pytest.skip("every wait was satisfied at its first poll")


@pytest.mark.parametrize("knob", ["FMD_PROJ_CHAIN", "FMD_DECODE_LAYERS"])
@pytest.mark.parametrize("prec", ["int8", "bf16"])
def test_fused_launch_modes_match_default(tmp_path, knob, prec):
    base = _run(tmp_path, {}, prec=prec)
    got = _run(tmp_path, {knob: "1"}, prec=prec)
    assert not got["errors"]
    assert got["logits"].shape == base["logits"].shape
    d = np.max(np.abs(got["logits"] - base["logits"]))
    assert d < TOL[prec], d


def test_projection_chain_full_widths(tmp_path):
    base = _run(tmp_path, {}, cfg="small", steps=3)
    got = _run(tmp_path, {"FMD_PROJ_CHAIN": "1"}, cfg="small", steps=3)
    assert not got["errors"]
    d = np.max(np.abs(got["logits"] - base["logits"]))
    assert d < TOL["int8"], d


@pytest.mark.parametrize("prec", ["bf16", "f16"])
def test_gemm_weight_staging_bit_identical(tmp_path, prec):
    base = _run(tmp_path, {}, cfg="small", prec=prec, mode="prefill")
    for v in ("0", "2"):
        got = _run(tmp_path, {"FMD_GEMM_BLDS": v}, cfg="small", prec=prec, mode="prefill")
        assert np.array_equal(got["logits"], base["logits"]), v
        assert np.array_equal(got["cache"], base["cache"]), v

"""C-ABI checks that need no GPU: the library loads, exports exactly what
include/fmd_dec.h declares, rejects bad arguments before touching a device,
and its host Q8_0 quantiser is bit-exact against the oracle."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]


def _declared():
    text = (ROOT / "include" / "fmd_dec.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fmd_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol(fmd):
    lib = fmd.lib()
    names = _declared()
    assert len(names) >= 25
    for n in names:
        assert hasattr(lib, n), n
    # and the Python binding table covers the header one-to-one
    from importlib import import_module

    dec = import_module("fast-moss-diarization_amd.decoder")
    assert sorted(dec.SIGNATURES) == names


def test_host_quantizer_bit_exact_vs_oracle(fmd, orc):
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((48, 1024)) * rng.uniform(1e-3, 3, (48, 1))).astype(np.float32)
    x[0, :32] = 0
    x[1, :32] = np.arange(32) - 15.5
    out = np.empty((48, 32, 34), dtype=np.uint8)
    rc = fmd.lib().fmd_quantize_q8_0(x.ctypes.data, 48, 1024, out.ctypes.data)
    assert rc == 0
    assert np.array_equal(out, orc.quantize_q8_0(x))


def test_bad_arguments_are_rejected_without_a_device(fmd):
    lib = fmd.lib()
    h = ctypes.c_void_p()
    assert lib.fmd_dec_create(None, 0, 0, 16, ctypes.byref(h)) == -1
    assert "null" in lib.fmd_last_error().decode()
    bad = fmd.TextConfig(vocab_size=64, hidden_size=256, intermediate_size=512,
                         num_hidden_layers=1, num_attention_heads=4, num_key_value_heads=2,
                         head_dim=64)
    c = bad.to_c()
    assert lib.fmd_dec_create(ctypes.byref(c), 0, 0, 16, ctypes.byref(h)) == -1
    assert "head_dim" in lib.fmd_last_error().decode()
    bad.head_dim, bad.hidden_size = 128, 200
    c = bad.to_c()
    assert lib.fmd_dec_create(ctypes.byref(c), 0, 0, 16, ctypes.byref(h)) == -1
    bad.hidden_size, bad.attention_bias = 256, True
    c = bad.to_c()
    assert lib.fmd_dec_create(ctypes.byref(c), 0, 0, 16, ctypes.byref(h)) == -1
    assert "attention_bias" in lib.fmd_last_error().decode()
    with pytest.raises(fmd.FmdError):
        fmd.Qwen3(bad, "bf16")


@pytest.mark.parametrize("name,want", [
    ("fp32", "F32"), ("F32", "F32"), ("float32", "F32"), ("full", "F32"),
    ("fp16", "F16"), ("half", "F16"), ("bf16", "BF16"), ("bfloat16", "BF16"),
    ("int8", "INT8"), ("q8_0", "INT8"), ("Q8", "INT8"), ("i8", "INT8"),
])
def test_precision_parse(fmd, name, want):
    """precision.rs:99-129."""
    assert fmd.Precision.parse(name) == fmd.Precision[want]


def test_precision_policy(fmd):
    P = fmd.Precision
    assert P.INT8.activation_dtype() == "f16" and P.INT8.is_quantized()
    assert P.BF16.activation_dtype() == "bf16" and not P.BF16.is_quantized()
    with pytest.raises(ValueError):
        P.parse("fp8")


def test_m0_check_accepts_copy_blocks_and_rejects_other_uses():
    """build.py's check of the device assembly: M0 appears only in the
    direct-to-LDS copy blocks of fmd_common.h's lds_copy16."""
    import importlib

    b = importlib.import_module("fast-moss-diarization_amd.build")
    ok = ("\tv_add_u32 v1, v2, v3\n\t;;#ASMSTART\n\ts_mov_b32 m0, s23\n\ts_nop 0\n"
          "\tglobal_load_lds_dwordx4 v13, s[18:19]\n\t;;#ASMEND\n")
    assert b.check_m0(ok * 3, "x") == 3
    for bad in ("\ts_mov_b32 m0, s4\n\tv_nop\n", "\ts_movk_i32 m0, 0x100\n",
                "\tv_readfirstlane_b32 s0, v1\n\ts_mov_b32 s1, m0\n"):
        with pytest.raises(RuntimeError, match="M0 used outside"):
            b.check_m0(ok + bad, "x")


def test_gelu_erf_approximation_constants_meet_the_published_bound():
    """gemm.hip's gelu_erf (Abramowitz & Stegun 7.1.26 for erfc, GELU as
    max(v, 0) - |v| erfc(|v|/sqrt 2)/2): its constants, read from the source,
    give |gelu - 0.5 v (1 + erf(v/sqrt 2))| <= |v| * 1.5e-7 / 2 (the published
    bound on erfc, halved) over a dense grid against math.erf in float64, and
    within 1e-6 * max(|v|, 1) in float32 arithmetic with the device's folded
    constants (exact reciprocal and exp2 standing in for the hardware's 1-ulp
    ones), on both sides of zero; the folded 1/sqrt 2 and -log2(e)/2 are
    checked against math."""
    import math

    src = (ROOT / "fast-moss-diarization_amd" / "csrc" / "gemm.hip").read_text()
    body = src[src.index("float gelu_erf(float v)"):]
    body = body[:body.index("\n}\n")]
    c = {k: float(v) for k, v in re.findall(r"\b(kP|kA[1-5]|kRsqrt2|kE)\s*=\s*(-?[0-9.]+)f", body)}
    assert sorted(c) == ["kA1", "kA2", "kA3", "kA4", "kA5", "kE", "kP", "kRsqrt2"]
    assert abs(c["kRsqrt2"] - 1.0 / math.sqrt(2.0)) < 1e-15
    assert abs(c["kE"] + 0.5 / math.log(2.0)) < 1e-15
    v = np.concatenate([np.linspace(-9.0, 9.0, 360001), [0.0, -0.0, 1e-30, -1e-30]])
    v32 = v.astype(np.float32)
    want = np.array([0.5 * x * (1.0 + math.erf(x / math.sqrt(2.0))) for x in v])
    want32 = np.array([0.5 * float(x) * (1.0 + math.erf(float(x) / math.sqrt(2.0))) for x in v32])

    def approx(v, ty, ps, ke):
        f = lambda x: ty(x)
        av = np.abs(v).astype(ty)
        t = (f(1.0) / (f(ps) * av + f(1.0))).astype(ty)
        p = f(0.5 * c["kA5"])
        for k in ("kA4", "kA3", "kA2", "kA1"):
            p = (t * p + f(0.5 * c[k])).astype(ty)
        h = ((t * p).astype(ty) * np.exp2((v * (v * f(ke)).astype(ty)).astype(ty)).astype(ty)).astype(ty)
        return (np.maximum(v, f(0.0)) - av * h).astype(np.float64)

    err = np.abs(approx(v, np.float64, c["kP"] / math.sqrt(2.0), -0.5 / math.log(2.0)) - want)
    assert bool(np.all(err <= np.abs(v) * 0.75e-7))
    # float32: the device folds p / sqrt 2 into one float constant; a few
    # roundings in h (< 1, 6e-8 each) and the hardware's 1-ulp reciprocal and
    # exp2 stay under 1e-6 relative, a few ulps of GELU's float32 value
    ps32 = np.float32(np.float32(c["kP"]) * np.float32(c["kRsqrt2"]))
    err32 = np.abs(approx(v32, np.float32, ps32, np.float32(c["kE"])) - want32)
    assert float(np.max(err32 / np.maximum(np.abs(v32).astype(np.float64), 1.0))) <= 1e-6

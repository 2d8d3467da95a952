"""fmd_op_attention_decode_noalloc (scratch in the library's static device
array, no allocation) against fmd_op_attention_decode (allocated workspace)
through the C ABI: the same context and the same appended K/V, bit for bit,
on two calls in a row -- the second with a smaller batch and a shorter
context -- for the single-launch kernel (16-bit) and the three-kernel path
(f32).  A call whose batch and capacity need more scratch than the array
holds fails with an error."""
import numpy as np
import pytest
import torch

from tests.gpu_util import small_cfg, tiny_cfg

pytestmark = pytest.mark.gpu

TDT = {"f32": torch.float32, "bf16": torch.bfloat16, "int8": torch.float16}


def _run(gpu, cfg, prec, B, ctx, seed, noalloc):
    rng = np.random.default_rng(seed)
    lens = rng.integers(max(1, ctx // 3), ctx + 1, B)
    L = int(lens.max())
    pad = (L - lens).astype(np.int32).tolist()
    kv = gpu.new_caches(B, L + 4)
    kv.fill_random(seed, L)
    g = torch.Generator().manual_seed(seed)
    qkv = torch.randn(B, cfg.q_dim() + 2 * cfg.kv_dim(), generator=g).to(TDT[prec]).cuda()
    out = torch.zeros(B, cfg.q_dim(), dtype=TDT[prec], device="cuda")
    fn = gpu.op_attention_decode_noalloc if noalloc else gpu.op_attention_decode
    # qkv and out are written on torch's stream, the op runs on the handle's own
    # stream: without this wait it could read qkv before the upload lands
    torch.cuda.synchronize()
    fn(kv, 1, qkv.data_ptr(), pad, B, out.data_ptr())
    torch.cuda.synchronize()
    k = kv.read(1, 0)[:, :, L]
    v = kv.read(1, 1)[:, :, L]
    return out.cpu(), k, v


@pytest.mark.parametrize("prec", ["int8", "bf16", "f32"])
def test_noalloc_attention_matches_allocating_op(fmd, prec):
    print(f"[gpu] no-alloc attention op {prec}", flush=True)
    cfg = small_cfg(fmd, layers=2, vocab=1024) if prec != "f32" else tiny_cfg(fmd, layers=2)
    gpu = fmd.Qwen3(cfg, prec, max_len=8192).load(fmd.synthetic_weights(cfg, seed=61))
    for B, ctx, seed in ((12, 3000, 62), (5, 700, 63)):
        want = _run(gpu, cfg, prec, B, ctx, seed, noalloc=False)
        got = _run(gpu, cfg, prec, B, ctx, seed, noalloc=True)
        assert torch.equal(got[0], want[0]), (B, ctx)
        assert np.array_equal(got[1], want[1]) and np.array_equal(got[2], want[2]), (B, ctx)
        assert torch.isfinite(got[0].float()).all()


def test_noalloc_attention_rejects_sizes_beyond_the_scratch(fmd):
    cfg = small_cfg(fmd, layers=1, vocab=1024)
    gpu = fmd.Qwen3(cfg, "int8", max_len=40000).load(fmd.synthetic_weights(cfg, seed=64))
    kv = gpu.new_caches(16, 32768)
    kv.fill_random(1, 100)
    qkv = torch.zeros(16, cfg.q_dim() + 2 * cfg.kv_dim(), dtype=torch.float16, device="cuda")
    out = torch.zeros(16, cfg.q_dim(), dtype=torch.float16, device="cuda")
    with pytest.raises(fmd.FmdError, match="bytes of scratch"):
        gpu.op_attention_decode_noalloc(kv, 0, qkv.data_ptr(), [0] * 16, 16, out.data_ptr())
    assert kv.len() == 100


@pytest.mark.parametrize("prec", ["int8", "f32"])
def test_noalloc_attention_under_graph_capture(fmd, prec):
    """The no-allocation op captured into a HIP graph on the handle's stream:
    its set-up (write position, pads, error word) travels as kernel arguments,
    so every replay -- with other eager work and synchronisations between the
    replays, and the captured host pad list gone -- gives the direct call's
    context and K/V rows bit for bit."""
    print(f"[gpu] no-alloc attention op under graph capture {prec}", flush=True)
    cfg = small_cfg(fmd, layers=2, vocab=1024) if prec != "f32" else tiny_cfg(fmd, layers=2)
    gpu = fmd.Qwen3(cfg, prec, max_len=8192).load(fmd.synthetic_weights(cfg, seed=65))
    B, ctx, seed = 7, 1500, 66
    want = _run(gpu, cfg, prec, B, ctx, seed, noalloc=True)
    rng = np.random.default_rng(seed)
    lens = rng.integers(max(1, ctx // 3), ctx + 1, B)
    L = int(lens.max())
    kv = gpu.new_caches(B, L + 4)
    kv.fill_random(seed, L)
    g = torch.Generator().manual_seed(seed)
    qkv = torch.randn(B, cfg.q_dim() + 2 * cfg.kv_dim(), generator=g).to(TDT[prec]).cuda()
    out = torch.zeros(B, cfg.q_dim(), dtype=TDT[prec], device="cuda")
    stream = torch.cuda.Stream()
    gpu.set_stream(stream.cuda_stream)
    graph = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with torch.cuda.graph(graph, stream=stream):
        gpu.op_attention_decode_noalloc(kv, 1, qkv.data_ptr(), (L - lens).astype(np.int32).tolist(),
                                        B, out.data_ptr())
    gpu.set_stream(None)
    torch.cuda.synchronize()
    # the capture itself ran nothing
    assert not out.any()
    other = torch.randn(4096, device="cuda")
    for rep in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.cpu(), want[0]), rep
        assert np.array_equal(kv.read(1, 0)[:, :, L], want[1]), rep
        assert np.array_equal(kv.read(1, 1)[:, :, L], want[2]), rep
        # eager work between replays: the allocating op on the same cache and
        # a torch reduction
        _run(gpu, cfg, prec, 3, 400, seed + rep + 1, noalloc=False)
        float(other.sum())
    del graph

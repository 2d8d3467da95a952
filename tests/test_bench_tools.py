"""The benchmark's rocprofv3 summarisers, on small synthetic CSV files (no GPU):
the derived counter columns and the per-launch split of one kernel's
dispatches."""
import csv

import pytest

import bench


def _write_counters(path, dispatches):
    """dispatches: (kernel name, work-groups, work-group size, {counter: value})."""
    rows = []
    for i, (name, wgs, wgsize, counters) in enumerate(dispatches, start=1):
        for c, v in counters.items():
            rows.append({"Dispatch_Id": i, "Correlation_Id": i, "Grid_Size": wgs * wgsize,
                         "Workgroup_Size": wgsize, "Kernel_Name": name,
                         "Counter_Name": c, "Counter_Value": v})
    path.mkdir(parents=True, exist_ok=True)
    with open(path / "run_counter_collection.csv", "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(rows[0]))
        w.writeheader()
        w.writerows(rows)


GEMM = "void gemm_dma_kernel<2, 5, 256, 3>(GemmArgs)"
NORM = "void layernorm16_kernel<2, 2>(void const*, int)"
ATTN = "void enc_attn_kernel<2>(EncAttnArgs)"


def _layer(valu_qkv, valu_out):
    # one encoder layer's order: LayerNorm, q|k|v GEMM, attention, out GEMM
    return [(NORM, 6004, 256, {"SQ_INSTS_VALU": 5.0, "SQ_INSTS_MFMA": 1.0}),
            (GEMM, 2304, 256, {"SQ_INSTS_VALU": valu_qkv, "SQ_INSTS_MFMA": 10.0}),
            (ATTN, 6144, 256, {"SQ_INSTS_VALU": 90.0, "SQ_INSTS_MFMA": 10.0}),
            (GEMM, 768, 256, {"SQ_INSTS_VALU": valu_out, "SQ_INSTS_MFMA": 10.0})]


def _derived(out):
    """{row label: valu_per_mfma} from the summariser's derived table."""
    lines = out.splitlines()
    start = next(i for i, l in enumerate(lines) if l.startswith("derived"))
    cols = lines[start][70:].split()
    res = {}
    for l in lines[start + 1:]:
        if l.strip():
            res[l[:70].rstrip()] = float(l[70:].split()[cols.index("valu_per_mfma")])
    return res


def test_counter_summary_splits_one_kernel_by_launch(tmp_path, capsys):
    _write_counters(tmp_path / "a", _layer(30.0, 20.0) + _layer(50.0, 40.0))
    bench.summarize_counters(tmp_path / "a", by_launch=True)
    d = _derived(capsys.readouterr().out)
    # the GEMM's two launch shapes get their own rows, each the mean of its
    # two dispatches; the first LayerNorm (no launch before it) ran once
    assert d["gemm_dma_kernel<2, 5, 256, 3> wgs 2304 < layernorm16_kernel 6004"] == pytest.approx(4.0)
    assert d["gemm_dma_kernel<2, 5, 256, 3> wgs 768 < enc_attn_kernel 6144"] == pytest.approx(3.0)
    assert d["enc_attn_kernel<2> wgs 6144 < gemm_dma_kernel 2304"] == pytest.approx(9.0)
    assert not any(k.startswith("layernorm16_kernel") for k in d)


def test_counter_summary_by_kernel_averages_every_launch(tmp_path, capsys):
    _write_counters(tmp_path / "b", _layer(30.0, 20.0) + _layer(50.0, 40.0))
    bench.summarize_counters(tmp_path / "b")
    d = _derived(capsys.readouterr().out)
    assert d["gemm_dma_kernel<2, 5, 256, 3>(GemmArgs)"] == pytest.approx(3.5)
    assert d["layernorm16_kernel<2, 2>(const*, int)"] == pytest.approx(5.0)


def test_mfma_busy_share_uses_one_xcds_cycles(tmp_path, capsys):
    # GRBM_GUI_ACTIVE sums 8 XCDs: 8000 -> 1000 cycles of the launch; 1024
    # SIMDs busy 512,000 cycles in total -> half of 1024 x 1000
    c = {"GRBM_GUI_ACTIVE": 8000.0, "SQ_VALU_MFMA_BUSY_CYCLES": 512000.0,
         "SQ_INSTS_VALU": 1.0, "SQ_INSTS_MFMA": 1.0}
    _write_counters(tmp_path / "c", [(GEMM, 768, 256, c), (GEMM, 768, 256, c)])
    bench.summarize_counters(tmp_path / "c")
    lines = capsys.readouterr().out.splitlines()
    start = next(i for i, l in enumerate(lines) if l.startswith("derived"))
    cols = lines[start][70:].split()
    row = next(l for l in lines[start + 1:] if l.startswith("gemm_dma_kernel"))
    assert float(row[70:].split()[cols.index("mfma_busy_%")]) == pytest.approx(50.0)


def test_trace_summary_per_launch(tmp_path, capsys):
    # kernel trace: per-dimension sizes, durations from the timestamps
    rows = []
    t = 0
    seq = [(NORM, (6004, 1, 1), 10), (GEMM, (2304, 1, 1), 100), (ATTN, (24, 16, 16), 300),
           (GEMM, (768, 1, 1), 60)] * 2
    for i, (name, grid, us) in enumerate(seq, start=1):
        rows.append({"Dispatch_Id": i, "Kernel_Name": name, "Start_Timestamp": t,
                     "End_Timestamp": t + us * 1000, "Workgroup_Size_X": 256,
                     "Workgroup_Size_Y": 1, "Workgroup_Size_Z": 1,
                     "Grid_Size_X": grid[0] * 256, "Grid_Size_Y": grid[1], "Grid_Size_Z": grid[2]})
        t += us * 1000 + 500
    (tmp_path / "t").mkdir()
    with open(tmp_path / "t" / "run_kernel_trace.csv", "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(rows[0]))
        w.writeheader()
        w.writerows(rows)
    bench.summarize_trace(tmp_path / "t")
    out = {l[:70].rstrip(): l[70:].split() for l in capsys.readouterr().out.splitlines()[1:]}
    assert out["enc_attn_kernel<2> wgs 6144 < gemm_dma_kernel 2304"][:2] == ["2", "300.00"]
    assert out["gemm_dma_kernel<2, 5, 256, 3> wgs 768 < enc_attn_kernel 6144"][:2] == ["2", "60.00"]
    assert out["gemm_dma_kernel<2, 5, 256, 3> wgs 2304 < layernorm16_kernel 6004"][:2] == ["2", "100.00"]

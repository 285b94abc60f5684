"""bench.py's profiler summaries on synthetic rocprofv3 CSVs (CPU only).

O-proj and FFN2 can run the same GEMM kernel on the same grid, so the
summaries label residual-GEMM dispatches by the kernel before them in the same
queue or stream; the roofline's HBM traffic is looked up with that label.
"""
import csv
import importlib.util
import os

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
_spec = importlib.util.spec_from_file_location("bench", os.path.join(ROOT, "bench.py"))
bench = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(bench)

K = "_ZN3bbh12_GLOBAL__N_1"
ATTN = K + "16attention_kernelILi2ELi1ELi3ELb0EEEvPKDF16_PKiPDF16_iiiiffPf"
LN = K + "12ln384_kernelEPKDF16_S2_S2_S2_PDF16_if"
QKV = K + "11gemm_kernelINS0_3CfgILi128ELi128ELi2ELi4ELi2ELi2ELi2EEELi0EEEvPKDF16_"
FFN1 = K + "11gemm_kernelINS0_3CfgILi64ELi64ELi2ELi2ELi2ELi4ELi2EEELi1EEEvPKDF16_"
RES = K + "11gemm_kernelINS0_3CfgILi64ELi64ELi2ELi2ELi4ELi0ELi2EEELi2EEEvPKDF16_"
LAYER = [(QKV, 110592), (ATTN, 98304), (RES, 73728), (LN, 196608), (FFN1, 294912), (RES, 73728),
         (LN, 196608)]


def _counter_csv(path, queues=(2, 3)):
    """Two layers per queue, queues interleaved dispatch by dispatch; O-proj
    fetches 100 KiB and FFN2 300 KiB."""
    rows, did = [], 0
    for _ in range(2):
        for i, (name, grid) in enumerate(LAYER):
            for q in queues:
                did += 1
                fetch = {2: 100.0, 5: 300.0}.get(i, 10.0)
                rows.append({"Dispatch_Id": did, "Queue_Id": q, "Grid_Size": grid, "Kernel_Name": name,
                             "Counter_Name": "FETCH_SIZE", "Counter_Value": fetch})
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(rows[0]))
        w.writeheader()
        w.writerows(rows)


def _trace_csv(path):
    """One layer on stream 4 (O-proj 6 us, FFN2 13 us), one on stream 1."""
    rows, did, t = [], 0, 1000
    for stream, scale in ((4, 1.0), (1, 1.5)):
        for i, (name, grid) in enumerate(LAYER):
            did += 1
            us = {2: 6.0, 5: 13.0}.get(i, 4.0) * scale
            rows.append({"Dispatch_Id": did, "Stream_Id": stream, "Kernel_Name": name,
                         "Start_Timestamp": t, "End_Timestamp": t + int(us * 1000),
                         "Grid_Size_X": grid, "Grid_Size_Y": 1, "Grid_Size_Z": 1})
            t += 20000
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(rows[0]))
        w.writeheader()
        w.writerows(rows)


def test_op_tags_split_shared_kernel_by_predecessor(tmp_path):
    p = tmp_path / "c.csv"
    _counter_csv(p)
    rows = list(csv.DictReader(open(p)))
    tags = bench.op_tags(rows, "Queue_Id", lambda r: int(r["Grid_Size"]))
    by_fetch = {}
    for r in rows:
        if r["Dispatch_Id"] in tags:
            by_fetch.setdefault(tags[r["Dispatch_Id"]], set()).add(float(r["Counter_Value"]))
    assert by_fetch == {" [o_proj]": {100.0}, " [ffn2]": {300.0}}
    # every residual GEMM dispatch got a tag; nothing else did
    res = {r["Dispatch_Id"] for r in rows if r["Kernel_Name"] == RES}
    assert set(tags) == res


def test_pmc_summary_and_traffic_rows_carry_the_op(tmp_path):
    c, t = tmp_path / "c.csv", tmp_path / "t.csv"
    _counter_csv(c)
    _trace_csv(t)
    table, rows = bench.pmc_summary([str(c)], str(t), 2.0, 1.0, "4")
    got = {r["kernel"]: r for r in rows if r["grid"] == 73728}
    assert set(got) == {"gemm_kernel<Cfg<64,64,2,2,4,0,2>, 2> [o_proj]",
                        "gemm_kernel<Cfg<64,64,2,2,4,0,2>, 2> [ffn2]"}
    assert got["gemm_kernel<Cfg<64,64,2,2,4,0,2>, 2> [o_proj]"]["read"] == 100.0 * 1024 * 2.0
    assert got["gemm_kernel<Cfg<64,64,2,2,4,0,2>, 2> [ffn2]"]["read"] == 300.0 * 1024 * 2.0
    assert got["gemm_kernel<Cfg<64,64,2,2,4,0,2>, 2> [o_proj]"]["us"] == 6.0  # stream 4 only
    assert got["gemm_kernel<Cfg<64,64,2,2,4,0,2>, 2> [ffn2]"]["us"] == 13.0
    assert "[ffn2]" in table


def test_trace_summary_means_per_stream(tmp_path):
    t = tmp_path / "t.csv"
    _trace_csv(t)
    table = bench.trace_summary(str(t), "4")
    line = [x for x in table.splitlines() if "[ffn2]" in x][0]
    cells = [x.strip() for x in line.strip("|").split("|")]
    assert cells[2:5] == ["2", "13.00", "19.50"]

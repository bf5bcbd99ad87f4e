"""bench.py's measurement helpers on synthetic profiler output (no GPU):
kernel naming, PMC byte scaling, the timed-dispatch selection from a kernel
trace, and the one-GPU contract."""
import csv
import json
import subprocess
import sys
from pathlib import Path

import pytest

import bench

ROOT = Path(__file__).resolve().parent.parent
COPY = "void pace_kv::(anonymous namespace)::page_copy_kernel<false, false, true>(pace_kv::(anonymous namespace)::CopyParams)"
COPY_T = COPY.replace("<false, false, true>", "<false, true, true>")


def write_csv(path, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(rows[0]))
        w.writeheader()
        w.writerows(rows)
    return str(path)


def test_copy_kernel_names_follow_the_store_policy():
    names = bench.copy_kernel_names("buffer", 65536)
    assert "page_copy_kernel<false, true, true> (pack, write-through stores)" in names
    assert "page_copy_kernel<false, false, true> (unpack" in names
    # 96 B: one partial row (a power of two); 3 KiB: three rows (not)
    assert bench.copy_kernel_names("fused", 96).startswith("page_copy_kernel<true, false, true> (move")
    assert bench.copy_kernel_names("fused", 3072).startswith("page_copy_kernel<false, false, false>")


def test_summarize_pmc_scales_counters_by_the_calibration_copy(tmp_path):
    gib_kib = float(1 << 20)
    # FETCH_SIZE reads half of the true bytes, WRITE_SIZE all of them: the
    # calibration copies of 1 GiB (the run's last three large copies) show it
    # and the factors undo it.  A 4 GiB copy earlier in the run and a 4 KiB
    # copy are not calibrations.
    cb = "__amd_rocclr_copyBuffer"
    fetch = [(COPY, 1000.0), (cb, 4 * gib_kib / 2), (COPY_T, 1000.0), (cb, 4.0)] + [(cb, gib_kib / 2)] * 3
    write = [(COPY, 2000.0), (cb, 4 * gib_kib), (COPY_T, 2000.0)] + [(cb, gib_kib)] * 3
    fetch = [{"Dispatch_Id": i + 1, "Kernel_Name": k, "Counter_Name": "FETCH_SIZE", "Counter_Value": v}
             for i, (k, v) in enumerate(fetch)]
    write = [{"Dispatch_Id": i + 1, "Kernel_Name": k, "Counter_Name": "WRITE_SIZE", "Counter_Value": v}
             for i, (k, v) in enumerate(write)]
    d = bench.summarize_pmc(write_csv(tmp_path / "f.csv", fetch), write_csv(tmp_path / "w.csv", write), "llama3-8b-512tok-fp16")
    assert d["fetch_scale"] == 2.0 and d["write_scale"] == 1.0     # the 4 KiB copy is not a calibration
    assert d["fetch_bytes_per_launch"] == 2000 * 1024
    assert d["write_bytes_per_launch"] == 2000 * 1024
    assert d["traffic_bytes_per_launch"] == 4000 * 1024
    assert d["fetch_dispatches"] == 2
    assert d["kernel"] == "page_copy_kernel<false, false, true> and page_copy_kernel<false, true, true>"


def test_summarize_pmc_needs_both_kinds_of_dispatch(tmp_path):
    rows = [{"Dispatch_Id": 1, "Kernel_Name": COPY, "Counter_Name": "FETCH_SIZE", "Counter_Value": 1.0}]
    path = write_csv(tmp_path / "f.csv", rows)
    with pytest.raises(SystemExit):
        bench.summarize_pmc(path, path, "llama3-8b-16req-bf16")


def test_pmc_markdown_states_algorithmic_bytes_per_layer_chunk(tmp_path):
    from paceserve_amd import workloads

    w = workloads.get("llama3-70b-256req-bf16")
    alg = 2 * 8 * w.n_pages * w.shape.page_bytes          # one launch = one 8-layer chunk
    t = {"workload": "llama3-70b-256req-bf16", "kernel": "page_copy_kernel<false, false, true>",
         "fetch_kib_per_dispatch_raw": 1.0, "fetch_calibration_kib_raw": 2.0, "fetch_scale": 2.0,
         "fetch_bytes_per_launch": alg // 2, "fetch_dispatches": 3, "write_kib_per_dispatch_raw": 1.0,
         "write_calibration_kib_raw": 1.0, "write_scale": 1.0, "write_bytes_per_launch": alg // 2,
         "write_dispatches": 3, "traffic_bytes_per_launch": alg}
    path = tmp_path / "t.json"
    path.write_text(json.dumps(t))
    md = bench.pmc_markdown(str(path))
    assert f"Algorithmic bytes per launch: {alg} (8 layers x {w.n_pages} pages" in md
    assert "= 1.00000 x algorithmic" in md
    assert "--workload llama3-70b-256req-bf16" in md


def test_timed_dispatches_skip_warmup_and_later_passes(tmp_path):
    # 2 warm-up steps and 3 timed steps of 2 launches, then 4 more launches;
    # page copies of another batch (a staging leg before, another workload
    # after) have another grid and are skipped
    cfg = {"pages": 10, "layers": 4, "payload_bytes": 4 * 10 * 65536}
    grid = 64 * 10 * 64
    rows, t = [], 0
    rows.append({"Dispatch_Id": 1, "Kernel_Name": COPY, "Start_Timestamp": 0, "End_Timestamp": 3,
                 "Grid_Size_X": 7 * 64})
    for i in range(2 * 2 + 3 * 2 + 4):
        dur = 10 if 4 <= i < 10 else 99
        rows.append({"Dispatch_Id": i + 2, "Kernel_Name": COPY, "Start_Timestamp": t,
                     "End_Timestamp": t + dur, "Grid_Size_X": grid})
        t += dur + 1
    rows.insert(3, {"Dispatch_Id": 100, "Kernel_Name": "other", "Start_Timestamp": 0, "End_Timestamp": 5,
                    "Grid_Size_X": grid})
    rows.append({"Dispatch_Id": 200, "Kernel_Name": COPY, "Start_Timestamp": t, "End_Timestamp": t + 1,
                 "Grid_Size_X": 3 * 64})
    path = write_csv(tmp_path / "k.csv", rows)
    b = {"warmup": 2, "steps": 3, "roofline": {"launches_per_step": 2}, "config": cfg}
    durs, span = bench.timed_dispatches(path, b)
    assert durs == [10] * 6
    assert span == 6 * 10 + 5


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in json.loads(r.stdout.strip().splitlines()[-1])["error"]


def test_summarize_promote_splits_the_inline_kernels(tmp_path):
    inline = "void pace_kv::(anonymous namespace)::page_copy_inline_kernel<false, {}, true, {}, {}>(x)"
    rows, t = [], 0
    for i, (pack, s_in, d_in, dur) in enumerate([("true", "true", "false", 150000),
                                                  ("false", "false", "true", 152000)] * 3
                                                 + [("false", "true", "true", 165000)] * 2):
        rows.append({"Dispatch_Id": i + 1, "Kernel_Name": inline.format(pack, s_in, d_in),
                     "Start_Timestamp": t, "End_Timestamp": t + dur})
        t += dur + 1000
    rows.append({"Dispatch_Id": 99, "Kernel_Name": COPY, "Start_Timestamp": 0, "End_Timestamp": 7})
    path = write_csv(tmp_path / "k.csv", rows)
    b = {"promote_4k": {"payload_bytes": 1 << 29, "buffer_native": {"p50_us": 327.0, "runs": 3},
                        "fused_native": {"p50_us": 186.0, "runs": 2}}}
    bj = tmp_path / "b.json"
    bj.write_text(json.dumps(b))
    md = bench.summarize_promote(path, str(bj), "CMD")
    assert "| pack (source ids inline) | 3 | 150.0 | 150.0 |" in md
    assert "| unpack (destination ids inline) | 3 | 152.0 | 152.0 |" in md
    assert "| move (both inline) | 2 | 165.0 | 165.0 |" in md
    assert "of which 302.0 us are the two kernels" in md and "of which 165.0 us is the move kernel" in md


def test_summarize_kernel_pmc_groups_by_kernel_and_grid(tmp_path):
    app = "void pace_kv::(anonymous namespace)::append_kernel<2, false, false, true>(pace_kv::(anonymous namespace)::AppendParams)"
    rows = []
    for i, (grid, val) in enumerate([(2097152, 100.0), (2097152, 300.0), (32768, 7.0)]):
        rows.append({"Dispatch_Id": i + 1, "Kernel_Name": app, "Grid_Size": grid, "Counter_Name": "FETCH_SIZE",
                     "Counter_Value": val})
    rows.append({"Dispatch_Id": 9, "Kernel_Name": "other", "Grid_Size": 64, "Counter_Name": "FETCH_SIZE",
                 "Counter_Value": 1.0})
    a = write_csv(tmp_path / "a.csv", rows)
    b = write_csv(tmp_path / "b.csv", [dict(r, Counter_Name="WRITE_SIZE", Counter_Value=2 * r["Counter_Value"])
                                       for r in rows])
    md = bench.summarize_kernel_pmc("append_kernel", "CMD1\nCMD2", [a, b])
    assert "CMD1\nCMD2" in md
    assert "| append_kernel<2, false, false, true> | 32768 | 1 | 7 | 14 |" in md
    assert "| append_kernel<2, false, false, true> | 2097152 | 2 | 200 | 400 |" in md
    assert "other" not in md


def test_tp8_share_is_the_70b_workload_with_one_kv_head():
    """One GPU's share at tensor parallelism 8 moves the same requests and
    block tables as the 70B workload, with 8 KiB pages (1 of 8 KV heads), so
    its payload is exactly an eighth."""
    from paceserve_amd import workloads

    full, share = workloads.get("llama3-70b-256req-bf16"), workloads.get("llama3-70b-256req-bf16-tp8")
    assert share.name in workloads.SHARDS and share.name not in workloads.NAMES
    assert share.src_tables == full.src_tables and share.lengths == full.lengths
    assert (share.src_pool_pages, share.dst_pool_pages) == (full.src_pool_pages, full.dst_pool_pages)
    assert share.shape.num_kv_heads * 8 == full.shape.num_kv_heads and share.shape.page_bytes == 8192
    assert share.payload_bytes * 8 == full.payload_bytes
    assert share.device_layers_per_chunk <= 64        # one launch per chunk

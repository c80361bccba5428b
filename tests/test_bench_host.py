"""CPU: bench.py's rocprofv3 summarizers on small synthetic CSVs -- launches grouped by kernel
and grid, each bench entry matched to its own group, the PMC traffic scaled by the 1 GiB copy
and read back by the roofline's lookup -- and the input-set rotation rule of its timing."""

import csv
import json

import bench

K = "void soupk::(anonymous namespace)::{}(int)"


def _write(path, header, rows):
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(header)
        w.writerows(rows)
    return str(path)


def _bench_json(tmp_path):
    line = {"kernels": {"rope_pack_fwd": {"kernel": "rope_pack_fwd_kernel", "us_mean": 5.0,
                                          "GBps": 6000.0, "frac_of_peak": 0.75, "bytes": 3000}},
            "kernels_other_shapes": {"rope_pack_fwd_ragged": {
                "kernel": "rope_pack_fwd_kernel", "us_mean": 4.0, "GBps": 4000.0,
                "frac_of_peak": 0.5, "bytes": 1000}},
            "launch_floor_us": {"empty_kernel_1wg": 4.0}}
    p = tmp_path / "bench.json"
    p.write_text("log line\n" + json.dumps(line) + "\n")
    return str(p)


def test_trace_groups_match_bench_entries(tmp_path):
    hdr = ["Dispatch_Id", "Kernel_Name", "Grid_Size_X", "Workgroup_Size_X", "Start_Timestamp",
           "End_Timestamp"]
    rows = []
    for i in range(4):      # the set's launches first, then the ragged shape's, then the floor
        rows.append([1 + i, K.format("rope_pack_fwd_kernel<64, false>"), 4096, 256, 0, 5000])
    for i in range(4):
        rows.append([10 + i, K.format("rope_pack_fwd_kernel<64, false>"), 2048, 256, 0, 4400])
    rows.append([20, K.format("bench_empty_kernel"), 256, 256, 0, 3900])
    out = bench.summarize_stats(_write(tmp_path / "t.csv", hdr, rows), _bench_json(tmp_path),
                                "cmd")
    lines = {ln.split("|")[1].strip(): ln for ln in out.splitlines() if ln.startswith("| ")}
    assert "| 4096 / 256 | 4 | 5.00 |" in lines["rope_pack_fwd"]
    assert "| 2048 / 256 | 4 | 4.40 |" in lines["rope_pack_fwd_ragged"]
    assert "1.100" in lines["rope_pack_fwd_ragged"]             # 4.40 / 4.00
    assert "0.975 (median)" in lines["launch floor: empty_kernel_1wg"]


def test_pmc_traffic_scaled_and_read_back(tmp_path):
    hdr = ["Dispatch_Id", "Kernel_Name", "Grid_Size", "Workgroup_Size", "Counter_Name",
           "Counter_Value"]
    gib = 1 << 20
    fetch = [[1, "__amd_rocclr_copyBuffer", 1, 1, "FETCH_SIZE", gib / 2],
             [2, K.format("rope_pack_fwd_kernel<64, false>"), 4096, 256, "FETCH_SIZE", 1.0],
             [3, K.format("rope_pack_fwd_kernel<64, false>"), 2048, 256, "FETCH_SIZE", 0.25]]
    write = [[1, "__amd_rocclr_copyBuffer", 1, 1, "WRITE_SIZE", gib],
             [2, K.format("rope_pack_fwd_kernel<64, false>"), 4096, 256, "WRITE_SIZE", 0.5],
             [3, K.format("rope_pack_fwd_kernel<64, false>"), 2048, 256, "WRITE_SIZE", 0.5]]
    table = bench.summarize_pmc(_write(tmp_path / "f.csv", hdr, fetch),
                                _write(tmp_path / "w.csv", hdr, write), _bench_json(tmp_path),
                                ["c1", "c2"])
    path = tmp_path / "traffic.md"
    path.write_text(table)
    assert bench.pmc_traffic("rope_pack_fwd", path) == 2560           # (1 x 2 + 0.5) KiB
    assert bench.pmc_traffic("rope_pack_fwd_ragged", path) == 1024    # (0.25 x 2 + 0.5) KiB
    assert bench.pmc_traffic("swiglu_bwd", path) is None


def test_trace_summary_groups_every_kernel(tmp_path):
    """summarize_trace: soupk and library kernels alike, grouped by (kernel, grid), in the order
    of first dispatch, device-side waits left out."""
    hdr = ["Dispatch_Id", "Kernel_Name", "Grid_Size_X", "Workgroup_Size_X", "Start_Timestamp",
           "End_Timestamp"]
    rows = [[1, K.format("bench_hold_kernel"), 64, 64, 0, 900000]]
    for i in range(3):
        rows.append([2 + i, K.format("gemm_tn_kernel<false>"), 65536, 256, 0, 20000 + 1000 * i])
    rows.append([5, "Cijk_Ailk_Bljk_HHS_BH_MT256x256x64(args)", 1024, 256, 0, 18000])
    rows.append([6, K.format("gemm_tn_kernel<false>"), 1024, 256, 0, 7000])
    rows.append([7, K.format("bench_hold_kernel"), 64, 64, 0, 900000])   # the next span:
    rows.append([8, K.format("gemm_tn_kernel<false>"), 65536, 256, 0, 9000])  # same grid
    trace = _write(tmp_path / "trace.csv", hdr, rows)
    text = bench.summarize_trace(trace, "title", "cmd")
    lines = [ln for ln in text.splitlines() if ln.startswith("| `")]
    assert len(lines) == 4 and "bench_hold" not in text
    assert lines[0].startswith("| `gemm_tn_kernel<false>` | 65536 / 256 | 3 | 21.00 | 21.00 |")
    assert lines[1].startswith("| `Cijk_Ailk_Bljk_HHS_BH_MT256x256x64` | 1024 / 256 | 1 | 18.00")
    assert lines[2].startswith("| `gemm_tn_kernel<false>` | 1024 / 256 | 1 | 7.00")
    assert lines[3].startswith("| `gemm_tn_kernel<false>` | 65536 / 256 | 1 | 9.00")


def test_rotation_sets_span_twice_the_infinity_cache():
    """Every timed kernel rotates through input sets whose inputs add up to at least 512 MB
    (twice the 256 MB Infinity Cache), and through at least 3; an explicit count overrides."""
    for in_bytes in (3_637_248, 8_388_608, 23_068_672, 77_791_232, 110_100_480, 622_329_856):
        n = bench.rotation_sets(in_bytes)
        assert n >= 3 and n * in_bytes >= bench.ROTATION_BYTES == 512 << 20
        assert n == 3 or (n - 1) * in_bytes < bench.ROTATION_BYTES      # no more than needed
    assert bench.rotation_sets(8_388_608, n_sets=2) == 2


def test_step_summary_reports_host_issue_time_of_the_slowest_step():
    """The per-step record names the slowest step and the host's issue time of it beside the
    median's, so an outlier can be attributed to the host (issue time up by about the step's
    excess) or to the device (issue time as usual)."""
    watch = bench.GcWatch()
    per = [600.0, 610.0, 1100.0, 605.0, 598.0]
    watch.host_us = [500.0, 505.0, 1010.0, 498.0, 502.0]
    st = bench.step_summary(per, sum(per), watch)
    assert st["slowest_step"] == 2 and st["max"] == 1100.0 and st["median"] == 605.0
    assert st["host_issue_slowest_step"] == 1010.0 and st["host_issue_median"] == 502.0
    assert st["mean"] == round(sum(per) / 5, 1) and st["gc_collections"] == 0
    plain = bench.step_summary(per, sum(per), bench.GcWatch())    # no host times recorded
    assert "host_issue_median" not in plain and plain["slowest_step"] == 2


def test_attention_block_steps_count_the_causal_key_blocks():
    """The attention counter table divides by the key-block steps a launch performs: a
    sequence of nb 64-row blocks has nb(nb+1)/2 (query block, key block) steps per head in the
    forward, and the backward's dK/dV and dQ workgroups walk that many each."""
    assert bench.attn_block_steps([64], 1) == (1, 2)
    assert bench.attn_block_steps([65], 1) == (3, 6)          # 2 blocks: (0,0), (1,0), (1,1)
    assert bench.attn_block_steps([512] * 4, 12) == (12 * 4 * 36, 2 * 12 * 4 * 36)
    assert bench.attn_block_steps([512, 152, 128, 96], 12) == (12 * (36 + 6 + 3 + 3),
                                                               2 * 12 * 48)
    assert bench.attn_block_steps([0, 1], 2) == (2, 4)
    # brute force over (query block, key block <= query block) pairs
    for n in (1, 63, 64, 200, 511):
        nb = -(-n // 64)
        pairs = sum(1 for q in range(nb) for k in range(q + 1))
        assert bench.attn_block_steps([n], 3) == (3 * pairs, 6 * pairs)


def test_nf4_resident_summary_reads_the_held_spans(tmp_path):
    """summarize_nf4_resident: the kernels between each odd and even device-side wait are one
    labelled segment, reported per step; launches outside the spans (warm-up) are left out."""
    hdr = ["Dispatch_Id", "Kernel_Name", "Grid_Size_X", "Workgroup_Size_X", "Start_Timestamp",
           "End_Timestamp"]
    hold = K.format("bench_hold_kernel")
    rows = [[1, K.format("gemm_tn_kernel<true>"), 64, 256, 0, 99000],       # warm-up
            [2, hold, 64, 64, 0, 1000],
            [3, K.format("gemm_tn_kernel<true>"), 64, 256, 0, 10000],
            [4, K.format("gemm_tn_kernel<true>"), 64, 256, 0, 12000],
            [5, K.format("split_sum_kernel"), 64, 256, 0, 2000],
            [6, hold, 64, 64, 0, 1000],
            [7, "Cijk_Alik_Bljk_HHS_BH_MT128x128x64(args)", 64, 256, 0, 50000],  # warm-up
            [8, hold, 64, 64, 0, 1000],
            [9, "Cijk_Alik_Bljk_HHS_BH_MT128x128x64(args)", 64, 256, 0, 8000],
            [10, hold, 64, 64, 0, 1000]]
    trace = _write(tmp_path / "trace.csv", hdr, rows)
    bj = tmp_path / "bench.json"
    bj.write_text(json.dumps({"nf4_resident_trace": [[16, "nf4", 2], [16, "unpacked", 1]]}) +
                  "\n")
    text = bench.summarize_nf4_resident(trace, str(bj), "cmd")
    assert "## 16 tokens, nf4 weights: 12.0 us of kernels per step" in text
    assert "| `gemm_tn_kernel<true>` | 1 | 11.0 |" in text
    assert "| `split_sum_kernel` | 0.5 | 1.0 |" in text
    assert "## 16 tokens, unpacked weights: 8.0 us of kernels per step" in text
    assert "99" not in text and "50.0" not in text

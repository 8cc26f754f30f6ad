"""bench.py's CPU-side pieces: the rocprofv3 summaries that turn counter and trace CSVs into the
committed profiles, checked on synthetic CSVs whose answers are known by construction, and the
contract's --gpus guard. No GPU: bench.py's functions are imported, not run."""
import csv
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402

GEMV = "void sn::(anonymous namespace)::gemv_kernel<{m}, 16>(sn::GemvArgs)"
COPY = "sn::(anonymous namespace)::copy_kernel(float const*, float*, unsigned long)"


def write_counters(path, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"])
        w.writeheader()
        for row in rows:
            w.writerow(dict(zip(["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"], row)))


def test_decode_counter_summary_recovers_known_bytes_and_rates(tmp_path):
    # Each measured GEMV dispatch reads exactly its algorithmic bytes (FETCH_SIZE reports half of
    # them, as for the calibration copy) and writes y, in a duration that gives 5 TB/s.
    launches = list(bench._decode_pmc_launches())
    fetch, write, trace = [], [], []
    fetch.append((1, COPY, "FETCH_SIZE", 1024 * 1024 // 2))  # 1 GiB copy: half reported
    write.append((1, COPY, "WRITE_SIZE", 1024 * 1024))
    for i, (m, _, k, n, _, _) in enumerate(launches):
        read = 4 * (k * n + m * k)
        fetch.append((i + 10, GEMV.format(m=m), "FETCH_SIZE", read / 2 / 1024))
        write.append((i + 10, GEMV.format(m=m), "WRITE_SIZE", 4 * m * n / 1024))
        ns = bench.decode_bytes(m, k, n) / 5000.0  # bytes / (5000 bytes per ns) = 5 TB/s
        trace.append((i + 10, GEMV.format(m=m), 1000, 1000 + ns))
    write_counters(tmp_path / "f.csv", fetch)
    write_counters(tmp_path / "w.csv", write)
    with open(tmp_path / "t.csv", "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Dispatch_Id", "Kernel_Name", "Start_Timestamp", "End_Timestamp"])
        for row in trace:
            w.writerow([row[0], row[1], row[2], int(round(row[3]))])
    text = bench.summarize_decode_pmc(str(tmp_path / "f.csv"), str(tmp_path / "w.csv"), str(tmp_path / "t.csv"), 1024)
    assert "factors 0.5000 (fetch), 1.0000 (write)" in text
    rows = [line.split() for line in text.splitlines() if line.strip().startswith("M=")]
    assert len(rows) == 15  # 3 row counts x 5 weights
    for r in rows:
        traffic_over_alg, alg_gbs, hbm_gbs = float(r[6]), float(r[8]), float(r[9])
        assert traffic_over_alg == pytest.approx(1.0, abs=2e-3)
        assert alg_gbs == pytest.approx(5000, rel=2e-3) and hbm_gbs == pytest.approx(5000, rel=5e-3)


def test_decode_counter_summary_rejects_a_mismatched_dispatch_count(tmp_path):
    write_counters(tmp_path / "f.csv", [(1, COPY, "FETCH_SIZE", 1), (2, GEMV.format(m=1), "FETCH_SIZE", 1)])
    write_counters(tmp_path / "w.csv", [(1, COPY, "WRITE_SIZE", 1), (2, GEMV.format(m=1), "WRITE_SIZE", 1)])
    with open(tmp_path / "t.csv", "w", newline="") as f:
        csv.writer(f).writerows([["Dispatch_Id", "Kernel_Name", "Start_Timestamp", "End_Timestamp"],
                                 [2, GEMV.format(m=1), 0, 10]])
    with pytest.raises(AssertionError):
        bench.summarize_decode_pmc(str(tmp_path / "f.csv"), str(tmp_path / "w.csv"), str(tmp_path / "t.csv"), 1024)


def test_counter_summary_derives_mfma_busy_and_waits(tmp_path):
    # Two dispatches of one kernel: MFMA busy = busy cycles / (4 x CU cycles), averaged.
    kernel = "void sn::(anonymous namespace)::causal_attention_kernel<64>(sn::(anonymous namespace)::AttentionArgs)"
    rows = []
    for d, (mfma, cu, wait, wave, valu, insts) in enumerate([(300, 100, 50, 100, 500, 100),
                                                             (300, 100, 70, 100, 700, 100)]):
        rows += [(d, kernel, "SQ_VALU_MFMA_BUSY_CYCLES", mfma), (d, kernel, "SQ_BUSY_CU_CYCLES", cu),
                 (d, kernel, "SQ_WAIT_INST_ANY", wait), (d, kernel, "SQ_WAVE_CYCLES", wave),
                 (d, kernel, "SQ_INSTS_VALU", valu), (d, kernel, "SQ_INSTS_MFMA", insts)]
    write_counters(tmp_path / "c.csv", rows)
    text = bench.summarize_counters([str(tmp_path / "c.csv")])
    assert "void causal_attention_kernel<64>" in text
    assert "MFMA busy 0.750; waiting 0.600; VALU per MFMA 5.00" in text


def test_counter_summary_of_the_nn_kernel_scales_by_the_copy(tmp_path):
    # The NN summary's copy calibration: FETCH_SIZE reports half, WRITE_SIZE all; every NN launch of
    # one step is listed, so the dispatch count must match the set's 49 forward products.
    nn = [s for _, layout, s in bench._set_specs() if layout == "NN"]
    fetch = [(1, COPY, "FETCH_SIZE", 1024 * 1024 // 2)]
    write = [(1, COPY, "WRITE_SIZE", 1024 * 1024)]
    for i, s in enumerate(nn):
        alg = 4 * (s.rows * s.inner + s.inner * s.cols + s.rows * s.cols)
        fetch.append((i + 5, bench.NN_KERNEL_KEY + "(Args)", "FETCH_SIZE", (alg - 4 * s.rows * s.cols) / 2 / 1024))
        write.append((i + 5, bench.NN_KERNEL_KEY + "(Args)", "WRITE_SIZE", 4 * s.rows * s.cols / 1024))
    write_counters(tmp_path / "f.csv", fetch)
    write_counters(tmp_path / "w.csv", write)
    text = bench.summarize_pmc(str(tmp_path / "f.csv"), str(tmp_path / "w.csv"), 1024)
    lines = {line.split(":")[0]: line.split(":")[1] for line in text.splitlines()
             if line.startswith(("traffic_bytes_per_launch", "algorithmic_bytes_per_launch"))}
    assert int(lines["traffic_bytes_per_launch"]) == pytest.approx(int(lines["algorithmic_bytes_per_launch"]), rel=1e-6)


def test_more_than_one_gpu_is_refused_with_a_message():
    out = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                         text=True, timeout=120)
    assert out.returncode == 2
    assert "one GPU" in out.stderr


def test_trace_summary_lists_kernels_and_compares_the_roofline_kernel(tmp_path):
    stats = tmp_path / "stats.csv"
    with open(stats, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Name", "Calls", "TotalDurationNs", "AverageNs", "Percentage", "MinNs", "MaxNs"])
        w.writerow([bench.NN_KERNEL_KEY + "(Args)", 49, 49 * 1_000_000, 1_000_000, 90.0, 900_000, 1_100_000])
        w.writerow(["void sn::(anonymous namespace)::fill_normal_kernel(float*)", 3, 30_000, 10_000, 10.0, 9_000, 11_000])
    line = tmp_path / "bench.json"
    line.write_text(json.dumps({"roofline": {"launch_ms_mean": 1.01}}) + "\n")
    text = bench.summarize_trace(str(stats), str(line))
    assert "fill_normal_kernel" in text
    assert "rocprof average 1.0000 ms over 49 launches; bench.py HIP-event mean 1.0100 ms (ratio 1.010)" in text


def test_kernel_counter_summary_recovers_known_bytes_and_rates(tmp_path):
    # Three decode-attention kernels, each reading 1.5x and writing 0.5x its algorithmic bytes in a
    # duration that gives 2 TB/s on the algorithmic bytes; FETCH_SIZE reports half of the bytes read.
    algorithmic = bench.decode_attention_algorithmic()
    names = {"decode_attention_kernel": "void sn::(anonymous namespace)::decode_attention_kernel<64, 1>(Args)",
             "gemv_nt_kernel": "void sn::(anonymous namespace)::gemv_nt_kernel<1>(Args)",
             "gemv_kernel": "void sn::(anonymous namespace)::gemv_kernel<1, 16>(Args)"}
    fetch, write = [(1, COPY, "FETCH_SIZE", 1024 * 1024 // 2)], [(1, COPY, "WRITE_SIZE", 1024 * 1024)]
    trace = []
    dispatch = 10
    for key, name in names.items():
        alg = algorithmic[key]
        for _ in range(4):
            fetch.append((dispatch, name, "FETCH_SIZE", 1.5 * alg / 2 / 1024))
            write.append((dispatch, name, "WRITE_SIZE", 0.5 * alg / 1024))
            trace.append((dispatch, name, 1000, 1000 + int(round(alg / 2000.0))))
            dispatch += 1
    write_counters(tmp_path / "f.csv", fetch)
    write_counters(tmp_path / "w.csv", write)
    with open(tmp_path / "t.csv", "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Dispatch_Id", "Kernel_Name", "Start_Timestamp", "End_Timestamp"])
        for row in trace:
            w.writerow([row[0], row[1], row[2], row[3]])
    text = bench.summarize_kernel_pmc(str(tmp_path / "f.csv"), str(tmp_path / "w.csv"), str(tmp_path / "t.csv"),
                                      1024, algorithmic)
    rows = {line.split()[0]: line.split() for line in text.splitlines()[3:] if line.strip()}
    assert set(rows) == set(names)
    for key, r in rows.items():
        assert int(r[1]) == 4
        assert float(r[5]) == pytest.approx(2.0, abs=2e-3)          # traffic / algorithmic
        assert float(r[7]) == pytest.approx(2000, rel=2e-3)         # algorithmic GB/s
        assert float(r[8]) == pytest.approx(4000, rel=2e-3)         # HBM GB/s


ROCMINFO = """*******
Agent 1
*******
  Name:                    AMD EPYC 9575F 64-Core Processor
  Marketing Name:          AMD EPYC 9575F 64-Core Processor
  Compute Unit:            128
  Max Clock Freq. (MHz):   3300
*******
Agent 2
*******
  Name:                    gfx950
  Marketing Name:          AMD Instinct MI355X
  Max Clock Freq. (MHz):   2400
  Compute Unit:            256
*******
Agent 3
*******
  Name:                    gfx950
  Compute Unit:            256
  Max Clock Freq. (MHz):   2100
"""


def test_device_peaks_come_from_the_first_gpu_agent():
    # The CPU agent is skipped; the first gfx9 agent's CU count and clock give the peaks.
    assert bench.parse_rocminfo_gpu(ROCMINFO) == (256, 2400)
    assert bench.parse_rocminfo_gpu(ROCMINFO.split("Agent 2")[0]) is None
    assert round(256 * 256 * 2400e6 / 1e12, 1) == bench.PEAK_FP32_TFLOPS

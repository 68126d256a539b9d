"""Host-side checks of bench.py's bookkeeping (no GPU): the byte models its roofline objects use,
the traffic figures it reads from the committed counter summaries, and the counter summarizer
that writes them. The timed workloads themselves need a GPU and run in the round-end bench."""
import csv
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402
from modelcore_amd import stats  # noqa: E402


def test_help_parses():
    out = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--help"],
                         capture_output=True, text=True, check=True).stdout
    for flag in ("--workload", "--decode-only", "--summarize-counters", "--summarize-pmc"):
        assert flag in out


def test_prefill_pass_bytes_is_the_sum_over_chunks():
    # 32 chunks of 512: chunk c reads its prefix (c + 1) * 512 keys of K and V per (row, KV head),
    # q once and writes out once; closed form of the sum.
    B, C, H, HKV, D, n = bench.PF_B, bench.PF_C, bench.PF_H, bench.PF_HKV, bench.D, bench.PF_T // bench.PF_C
    kv = B * HKV * D * 2 * 2 * C * n * (n + 1) // 2
    qo = n * 2 * B * C * H * D * 2
    assert bench.prefill_pass_bytes() == kv + qo


def test_mixed_step_bytes_matches_the_byte_model():
    want = 0
    for i in range(bench.MX_LAYERS):
        w = -1 if i % 4 == 3 else bench.MX_WIN
        want += stats.decode_step_bytes([bench.MX_P + 3] * bench.MX_B, bench.MX_H, bench.MX_HKV,
                                        bench.D, 2, window=w)
    assert bench.mixed_step_bytes(3, 1) == want


@pytest.mark.parametrize("name", sorted(bench.TRAFFIC_PROFILES))
def test_committed_traffic_summaries_are_read_and_scaled(name):
    spec = bench.TRAFFIC_PROFILES[name]
    with open(os.path.join(ROOT, spec["file"])) as f:
        text = f.read()
    algo = int(text.split("algorithmic_bytes_per_unit:")[1].split()[0])
    traffic = int(text.split("traffic_bytes_per_unit:")[1].split()[0])
    t, src = bench.profile_traffic(name, algo)
    assert t == traffic and spec["file"] in src
    t2, src2 = bench.profile_traffic(name, 2 * algo)  # other positions: scaled by the ratio
    assert t2 == round(traffic / algo * 2 * algo) and "scaled" in src2
    assert 1.0 <= traffic / algo < 2.0, "measured traffic within 2x of the algorithmic bytes"


def _write_counters(path, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"])
        w.writeheader()
        for r in rows:
            w.writerow(r)


def test_summarize_counters_scales_by_the_copy_calibration(tmp_path, capsys):
    copy_kib = bench.COPY_BYTES / 1024
    _write_counters(tmp_path / "cf.csv", [dict(Dispatch_Id=1, Kernel_Name="__amd_rocclr_copyBuffer",
                                               Counter_Name="FETCH_SIZE", Counter_Value=copy_kib / 2)])
    _write_counters(tmp_path / "cw.csv", [dict(Dispatch_Id=1, Kernel_Name="__amd_rocclr_copyBuffer",
                                               Counter_Name="WRITE_SIZE", Counter_Value=copy_kib)])
    # Two launches of the replication kernel, the last one counted: 100 KiB fetched (x 2 after
    # calibration) and 300 KiB written.
    _write_counters(tmp_path / "f.csv", [
        dict(Dispatch_Id=5, Kernel_Name="kv_replicate_kernel<x>", Counter_Name="FETCH_SIZE", Counter_Value=7),
        dict(Dispatch_Id=9, Kernel_Name="kv_replicate_kernel<x>", Counter_Name="FETCH_SIZE", Counter_Value=100)])
    _write_counters(tmp_path / "w.csv", [
        dict(Dispatch_Id=5, Kernel_Name="kv_replicate_kernel<x>", Counter_Name="WRITE_SIZE", Counter_Value=1),
        dict(Dispatch_Id=9, Kernel_Name="kv_replicate_kernel<x>", Counter_Name="WRITE_SIZE", Counter_Value=300)])
    bench.summarize_counters("replicate", str(tmp_path / "f.csv"), str(tmp_path / "w.csv"),
                             str(tmp_path / "cf.csv"), str(tmp_path / "cw.csv"), 1, 500 * 1024)
    out = capsys.readouterr().out
    assert f"traffic_bytes_per_unit: {(2 * 100 + 300) * 1024}" in out
    assert f"algorithmic_bytes_per_unit: {500 * 1024}" in out


def test_summarize_pmc_takes_the_last_dispatches(tmp_path, capsys):
    _write_counters(tmp_path / "p.csv", [
        dict(Dispatch_Id=d, Kernel_Name="prefill_mfma_kernel(...)", Counter_Name="SQ_WAVES",
             Counter_Value=v) for d, v in ((1, 1000), (2, 10), (3, 30))])
    bench.summarize_pmc([str(tmp_path / "p.csv")], "prefill_mfma_kernel", 2)
    assert "| SQ_WAVES | 20 |" in capsys.readouterr().out


def test_sample_step_bytes_counts_weights_and_the_shared_prompt_once():
    # bf16 weights: 32 layers of QKV stack (6144 x 4096), c_proj (4096 x 4096), gate/up and
    # down_proj (3 x 14336 x 4096) = 32 x 218 103 808 elements, plus the 32768 x 4096 lm_head.
    assert bench.sample_weight_bytes() == 2 * (32 * 218_103_808 + 32768 * 4096) == 14_227_079_168
    # One decode step at decode step `first`: each row's own keys past the prompt (the new
    # token's K/V counted as read and written), q and out, plus the prompt's K/V once per layer.
    first, P = 7, bench.SM_PROMPT
    own = stats.decode_step_bytes([P + first - P] * bench.SM_ROWS, bench.SM_H, bench.SM_HKV,
                                  bench.D, 2)
    prompt = 2 * P * bench.SM_HKV * bench.D * 2
    assert bench.sample_step_bytes(first, 1) == bench.sample_weight_bytes() + \
        (own + prompt) * bench.SM_LAYERS
    # Without the shared prompt: every row's K/V (the reference's byte model).
    every = stats.decode_step_bytes([P + first] * bench.SM_ROWS, bench.SM_H, bench.SM_HKV,
                                    bench.D, 2)
    assert bench.sample_step_bytes(first, 1, shared=0) == bench.sample_weight_bytes() + \
        every * bench.SM_LAYERS

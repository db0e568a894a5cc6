"""perf.harness's result log on the CPU: check() semantics (float64,
atol + rtol * |ref|, NaN fails) and one log_result record written and read
back (the reference's bench/harness.py:62-91)."""
import json

import torch

import perf.harness as harness


def test_check_passes_within_tolerance_and_fails_on_nan():
    ref = torch.tensor([1.0, -2.0, 0.0, 1e-3])
    ok = harness.check(ref + torch.tensor([1e-6, -1e-6, 5e-6, 0.0]), ref, atol=1e-5, rtol=1e-4)
    assert ok.passed and abs(ok.max_abs - 5e-6) < 1e-9 and abs(ok.cosine - 1.0) < 1e-9
    bad = harness.check(ref + torch.tensor([0.0, 0.0, 2e-5, 0.0]), ref, atol=1e-5, rtol=1e-4)
    assert not bad.passed and abs(bad.max_abs - 2e-5) < 1e-9
    # the relative term: |diff| = 1e-4 passes at |ref| = 2 with rtol 1e-4
    assert harness.check(torch.tensor([2.0 + 1e-4]), torch.tensor([2.0]), atol=1e-5, rtol=1e-4).passed
    nan = harness.check(torch.tensor([float("nan"), 1.0]), torch.tensor([0.0, 1.0]))
    assert not nan.passed


def test_log_result_appends_jsonl(tmp_path, monkeypatch):
    monkeypatch.setattr(harness, "RESULTS_DIR", tmp_path)
    s = harness.Samples([0.3, 0.1, 0.2])
    c = harness.check(torch.ones(3), torch.ones(3))
    path = harness.log_result("attention_train", {"batch": 8, "seq_len": 1024}, timing=s, check=c, value=491.5)
    harness.log_result("attention_train", {"batch": 4}, value=1.0)
    lines = path.read_text().splitlines()
    assert path == tmp_path / "attention_train.jsonl" and len(lines) == 2
    rec = json.loads(lines[0])
    assert rec["config"] == {"batch": 8, "seq_len": 1024} and rec["value"] == 491.5
    assert rec["timing"]["median_ms"] == 0.2 and rec["timing"]["n_iters"] == 3
    assert rec["check"]["passed"] is True and rec["env"]["torch"] == torch.__version__
    assert rec["time"].endswith("+00:00")
    assert json.loads(lines[1])["timing"] is None

"""bench.py's contract pieces that run without a GPU: the one-GPU refusal,
the kernel names it reports, and the committed traffic it attaches."""

from __future__ import annotations

import json
import subprocess
import sys
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402


def test_more_than_one_gpu_is_refused():
    proc = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                          cwd=ROOT, timeout=300)
    assert proc.returncode == 2, proc.stderr
    line = json.loads(proc.stdout.strip().splitlines()[-1])
    assert "one GPU" in line["error"] and line["gpus_requested"] == 2


def test_kernel_labels_are_the_device_symbols():
    assert bench.kernel_label("factor_stream", 1) == "k_factor_stream_bf16<1>"
    assert bench.kernel_label("factor_stream", 3) == "k_factor_stream_bf16<3>"
    assert bench.kernel_label("project", (torch.bfloat16, 2)) == "k_project_stream_bf16<2>"
    assert bench.kernel_label("project", (torch.float32, 1)) == "k_project_f32"
    assert bench.kernel_label("factor", (torch.bfloat16, 3)) == "k_factor_bf16<3>"
    assert bench.kernel_label("factor", (torch.float32, 1)) == "k_factor_f32"
    assert bench.kernel_label("factor_project", None) == "k_factor_project_bf16"
    assert bench.kernel_label("planes", None) == "k_pack_planes"
    assert bench.kernel_label("scale_sum", None) == "k_scale_sum"
    assert bench.kernel_label("lin_norm", 0) == "k_lin_outer_norm"
    assert bench.kernel_label("lin_norm", 2) == "k_lin_gram2_norm"
    assert bench.kernel_label("lin_sum", 0) == "k_lin_clip_sum<true>"
    assert bench.kernel_label("lin_sum", None) == "k_lin_clip_sum<false>"
    assert bench.kernel_label("lin_moments", 1) == "k_lin_moments_guarded"


def test_committed_traffic_matches_on_design_bytes_only():
    data = json.loads((ROOT / "profiles" / "traffic.json").read_text())
    label = "k_factor_stream_bf16<1>"
    entry = data["kernels"][label]
    assert bench.committed_traffic(label, entry["algorithmic_bytes"]) == entry["traffic_bytes"]
    assert bench.committed_traffic(label, entry["algorithmic_bytes"] + 1) is None
    assert bench.committed_traffic("k_no_such_kernel", 1) is None
    # The committed summary is of the launch the C3 roofline names, within
    # a few percent of its design bytes (the streaming minimum).
    assert 1.0 <= entry["traffic_bytes"] / entry["algorithmic_bytes"] < 1.05


def test_cpu_model_is_named():
    name = bench.cpu_model()
    assert isinstance(name, str) and name

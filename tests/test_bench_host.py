"""bench.py's host rows (--config quant, --config tokenizer) on the CPU: one
short run each prints one JSON line whose parity fields hold (quantized
expert blocks equal to the numpy restatement's; encoded lines equal to the
pure-Python restatement's) and whose throughput and CPU baseline are set."""
from __future__ import annotations

import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def run_bench(config):
    out = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--config", config,
                          "--steps", "1", "--warmup", "0", "--cpu-seconds", "0.5"],
                         cwd=ROOT, capture_output=True, text=True, timeout=600)
    assert out.returncode == 0, out.stderr[-2000:]
    return json.loads(out.stdout.strip().splitlines()[-1])


def test_bench_quant_line():
    line = run_bench("quant")
    assert line["unit"] == "layers/s" and line["value"] > 0 and line["n_gpus"] == 0
    assert line["parity"]["expert_blocks_equal_oracle"] is True
    assert line["cpu_baseline"]["kind"] == "port" and line["cpu_baseline"]["value"] > 0


def test_bench_tokenizer_line():
    pytest.importorskip("tokenizers")
    line = run_bench("tokenizer")
    assert line["unit"] == "MiB/s" and line["value"] > 0 and line["sentencepiece_mib_s"] > 0
    assert line["parity"] == {"byte_level_lines_equal_oracle": True,
                              "sentencepiece_lines_equal_oracle": True}
    assert line["cpu_baseline"]["value"] > 0

"""CPU checks of bench.py's reporting helpers (no GPU): the algorithmic work
behind roofline.achieved, the staleness guard of the committed HBM-traffic
record, and the one-GPU contract."""
import hashlib
import json
import os
import shutil
import subprocess
import sys

import bench

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_roofline_work_config3():
    # B=1, H=8, N=29,952 -> Mb = 468 query blocks, Np = 468, T = 46, no prefix tail
    pairs, ops_i8, flops16 = bench.roofline_work(1, 8, 468, 46, 0, True)
    assert pairs == 8 * 468 * 46 == 172_224
    assert ops_i8 == pairs * 2 * 64 ** 3 == 90_294_976_512
    assert flops16 == 5 * ops_i8 == 451_474_882_560
    # roofline time: int8 at 5.0 POP/s plus 16-bit at 2.5 PFLOP/s
    t_roof = ops_i8 / (bench.PEAK_I8_TOPS * 1e12) + flops16 / (bench.PEAK_BF16_TFLOPS * 1e12)
    assert abs(t_roof * 1e6 - 198.65) < 0.01
    # primal only: one 16-bit product per pair
    assert bench.roofline_work(1, 8, 468, 46, 0, False)[2] == ops_i8


def test_measured_traffic_only_for_the_measured_source(tmp_path, monkeypatch):
    rec_path = os.path.join(ROOT, "profiles", "fwd_jvp_config3_traffic.json")
    with open(rec_path) as f:
        rec = json.load(f)
    with open(os.path.join(ROOT, rec["source"]), "rb") as f:
        current = hashlib.sha256(f.read()).hexdigest() == rec["source_sha256"]
    # the figure is reported exactly while the record matches the kernel source
    assert bench.measured_traffic(3, True) == (rec["bytes_per_launch"] if current else None)
    assert bench.measured_traffic(2, False) is None
    assert bench.measured_traffic(3, False) is None
    # the same record next to an edited kernel source is stale: no figure
    (tmp_path / "profiles").mkdir()
    shutil.copy(rec_path, tmp_path / "profiles")
    src = tmp_path / rec["source"]
    src.parent.mkdir(parents=True)
    src.write_bytes(open(os.path.join(ROOT, rec["source"]), "rb").read() + b"\n// edited\n")
    monkeypatch.setattr(bench, "ROOT", str(tmp_path))
    assert bench.measured_traffic(3, True) is None


def test_more_than_one_gpu_is_refused():
    res = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                         capture_output=True, text=True, timeout=300)
    assert res.returncode != 0
    assert "one GPU" in res.stderr and res.stdout.strip() == ""

"""The C runtime's host code (loader, planner, operator operand reading) under
AddressSanitizer and UBSan, on the CPU.

`spinn_load` parses untrusted files, as the reference's does
(SPINN/run_time/spinn_runtime.c:21-124). This builds runtime.c, planner.c and
ops.c with gcc -fsanitize=address,undefined over a host-memory stand-in for the
device layer (tests/hostsan/hip_stub.c) and drives load -> plan -> run -> free
over generated models and corrupted copies of them: truncations at every
section boundary, flipped bytes in the header, tensor and node tables, and
out-of-range ids, dims and sizes. Every file must either be rejected or go
through cleanly; any sanitizer report fails the test.
"""
import os
import random
import shutil
import struct
import subprocess
from pathlib import Path

import pytest

from spinn_amd import ennf as E
from spinn_amd import models

ROOT = Path(__file__).resolve().parents[1]
HOST = ROOT / "spinn_amd" / "csrc" / "host"
SAN = ROOT / "tests" / "hostsan"


@pytest.fixture(scope="module")
def san_bin(tmp_path_factory):
    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    out = tmp_path_factory.mktemp("hostsan") / "load_plan_run"
    cmd = ["gcc", "-g", "-O1", "-std=gnu11", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           "-fno-omit-frame-pointer", f"-I{ROOT / 'include'}", f"-I{HOST}",
           str(HOST / "runtime.c"), str(HOST / "planner.c"), str(HOST / "ops.c"),
           str(SAN / "hip_stub.c"), str(SAN / "load_plan_run.c"), "-lm", "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0 and "asan" in (r.stderr + r.stdout).lower():
        pytest.skip("sanitizer runtime not available: " + r.stderr[-300:])
    assert r.returncode == 0, r.stderr[-3000:]
    return out


def _run(binary, files):
    env = dict(os.environ)
    env["ASAN_OPTIONS"] = "detect_leaks=1:abort_on_error=0:exitcode=86"
    env["UBSAN_OPTIONS"] = "print_stacktrace=1:halt_on_error=1:exitcode=87"
    env.pop("SPINN_PROFILE", None)
    r = subprocess.run([str(binary), *map(str, files)], capture_output=True, text=True, env=env, timeout=600)
    report = r.stderr
    assert r.returncode == 0 and "ERROR: AddressSanitizer" not in report and "runtime error" not in report, (
        f"rc={r.returncode}\n{report[-4000:]}")
    return r.stdout.splitlines()


def _models(tmp):
    paths = []
    g, _ = models.resnet(batch=2, seed=1, blocks=(1, 1, 1, 1), hw=32, num_classes=10)
    paths.append(g.write(tmp / "resnet.ennf"))
    g, _ = models.yolov10n(batch=1, seed=2, hw=64)
    paths.append(g.write(tmp / "yolo.ennf"))
    g, _ = models.gemm_model(m=4, n=8, k=16, seed=3)
    paths.append(g.write(tmp / "gemm.ennf"))
    return paths


def test_valid_models_run_clean(san_bin, tmp_path):
    paths = _models(tmp_path)
    lines = _run(san_bin, paths)
    assert len(lines) == len(paths)
    for line in lines:
        assert "load=ok plan=0 run=0" in line, line


def test_plan_folds_on_host(san_bin, tmp_path, monkeypatch):
    """The plan step's folds, decided on host addresses (the stand-in's arena): YOLOv10n's
    attention has a Transpose read only by a MatMul and a scalar Mul of a MatMul's product,
    both folded; SPINN_PLAN_FOLD=0 folds nothing; either way load, plan and run are clean."""
    g, _ = models.yolov10n(batch=1, seed=4, hw=64)
    path = g.write(tmp_path / "yolo_fold.ennf")
    line = _run(san_bin, [path])[0]
    fields = dict(f.split("=") for f in line.split()[1:])
    assert fields["plan"] == "0" and fields["run"] == "0", line
    assert int(fields["transposes"]) >= 1 and int(fields["scales"]) == 1, line
    monkeypatch.setenv("SPINN_PLAN_FOLD", "0")
    line = _run(san_bin, [path])[0]
    fields = dict(f.split("=") for f in line.split()[1:])
    assert fields["run"] == "0" and fields["views"] == "0" and fields["transposes"] == "0" and fields["scales"] == "0"


def test_corrupted_files_are_rejected_or_clean(san_bin, tmp_path):
    rng = random.Random(1234)
    srcs = _models(tmp_path)
    cases = []
    for si, src in enumerate(srcs):
        blob = Path(src).read_bytes()
        hdr = E.read(blob)["header"]
        head = min(len(blob), hdr["weight_data_offset"])  # header, tables and parameters
        # truncations: inside the header and at / around every table's start
        cuts = {8, 40, 63, 64, 65, len(blob) // 2, len(blob) - 4}
        for k in ("graph_meta_offset", "node_table_offset", "tensor_meta_offset", "weight_data_offset"):
            cuts.update({hdr[k] - 1, hdr[k], hdr[k] + 1, hdr[k] + 30})
        cuts = sorted(cuts)
        for c in cuts:
            if 0 < c < len(blob):
                p = tmp_path / f"m{si}_cut{c}.ennf"
                p.write_bytes(blob[:c])
                cases.append(p)
        # byte flips in the first 4 KB (header, tensor / node tables, params)
        for t in range(60):
            b = bytearray(blob)
            for _ in range(rng.choice([1, 2, 4, 8])):
                i = rng.randrange(4, max(5, head))  # keep the magic so the parse goes deep
                b[i] = rng.choice([0x00, 0xFF, 0x7F, 0x80, rng.randrange(256)])
            p = tmp_path / f"m{si}_flip{t}.ennf"
            p.write_bytes(bytes(b))
            cases.append(p)
        # 32-bit fields forced to extreme values at every 4-byte slot of the header
        for off in range(4, 64, 4):
            for val in (0xFFFFFFFF, 0x7FFFFFFF, 0x80000000, len(blob) + 1):
                b = bytearray(blob)
                struct.pack_into("<I", b, off, val)
                p = tmp_path / f"m{si}_hdr{off}_{val:x}.ennf"
                p.write_bytes(bytes(b))
                cases.append(p)
    lines = _run(san_bin, cases)
    assert len(lines) == len(cases)
    rejected = sum("load=fail" in l or "plan=-" in l for l in lines)
    # the corruptions must be noticed somewhere (not all of them: some flips hit
    # bytes no reader looks at)
    assert rejected >= len(cases) // 4, f"only {rejected} of {len(cases)} corrupted files rejected"

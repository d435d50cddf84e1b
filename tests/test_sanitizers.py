"""CPU tier: libmiattn's GGUF loader and the CPU oracle built with
AddressSanitizer + UBSan (tests/san/), any report fatal.  The loader walks a
valid file, the malformed files of test_gguf.py, every 97th truncation of the
valid file and 64 seeded byte corruptions of it; the oracle driver calls each
oracle entry point on small shapes (wrapped rings, a slot written twice, a
negative position)."""

import os
import shutil
import subprocess

import numpy as np
import pytest

import _gguf as W
import _oracle as O

SAN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "san")
ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0",
           UBSAN_OPTIONS="print_stacktrace=1")


@pytest.fixture(scope="module")
def drivers():
    if shutil.which("gcc") is None:
        pytest.skip("no gcc")
    r = subprocess.run(["make", "-C", SAN], capture_output=True, text=True)
    if r.returncode != 0:
        if "fsanitize" in r.stderr and "cannot find" in r.stderr:
            pytest.skip("sanitizer runtimes not installed")
        raise AssertionError(r.stdout + r.stderr)
    return os.path.join(SAN, "_build", "gguf_walk"), os.path.join(SAN, "_build", "oracle_run")


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True, env=ENV, timeout=300)
    report = ("ERROR: AddressSanitizer" in r.stderr) or ("runtime error:" in r.stderr)
    return r, report


def test_gguf_loader_under_sanitizers(tmp_path, drivers):
    walk, _ = drivers
    g = np.random.default_rng(3)
    meta, tensors = W.mistral_like(g, q4_maker=O.make_q4_0)
    good = tmp_path / "good.gguf"
    offs = W.write(good, meta, tensors)
    blob = good.read_bytes()
    files = [good]
    for name, data in W.malformed_variants(blob, offs["__data__"]).items():
        files.append(tmp_path / f"bad_{name}.gguf")
        files[-1].write_bytes(data)
    files.append(tmp_path / "bad_offset.gguf")
    W.bad_offset_file(files[-1])
    for n in range(0, len(blob), 97):
        files.append(tmp_path / f"cut_{n}.gguf")
        files[-1].write_bytes(blob[:n])
    rng = np.random.default_rng(11)
    head = offs["__data__"]  # corrupt the header, metadata and tensor records
    for i in range(64):
        b = bytearray(blob)
        for _ in range(1 + i % 4):
            b[int(rng.integers(0, head))] = int(rng.integers(0, 256))
        files.append(tmp_path / f"flip_{i}.gguf")
        files[-1].write_bytes(bytes(b))
    files.append(tmp_path / "missing.gguf")
    r, report = _run([walk] + [str(f) for f in files])
    assert not report, r.stderr[-4000:]
    assert r.returncode == 0, r.stdout[-4000:] + r.stderr[-2000:]
    lines = [l for l in r.stdout.splitlines() if not l.startswith("  ")]
    assert len(lines) == len(files)
    status = {os.path.basename(l.split()[0]): int(l.split()[1]) for l in lines}
    assert status["good.gguf"] == 0
    for name in list(W.malformed_variants(blob, offs["__data__"])) + ["offset"]:
        assert status[f"bad_{name}.gguf"] != 0, name
    assert status["missing.gguf"] != 0


def test_oracle_under_sanitizers(drivers):
    _, orun = drivers
    r, report = _run([orun])
    assert not report, r.stderr[-4000:]
    assert r.returncode == 0 and "all finite" in r.stdout, r.stdout + r.stderr[-2000:]

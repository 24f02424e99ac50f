"""The .ssm reader and writer under AddressSanitizer + UndefinedBehaviorSanitizer
(host side only, CPU): tests/cpp/_bin/ssm_asan opens every corrupted file of
test_ssm_file.CASES, a few hundred randomly mutated headers / indexes /
truncations of a valid file and of a writer-made model, walks what it
accepts and must finish with no sanitizer report.  The messages of the
rejected CASES files are checked as in test_ssm_file."""
import os
import re
import subprocess

import numpy as np
import pytest

from test_ssm_file import CASES, py_write, small_tensors

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "_bin", "ssm_asan")
ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=0",
           UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")


@pytest.fixture(scope="module")
def asan_bin():
    if not os.path.exists(BIN):
        r = subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "tests", "cpp"), "asan"],
                           capture_output=True, text=True)
        if r.returncode != 0:
            pytest.fail("building the sanitizer driver failed:\n" + r.stdout[-2000:] + r.stderr[-2000:])
    return BIN


def _run(bin_, args):
    r = subprocess.run([bin_, *args], capture_output=True, text=True, errors="replace", env=ENV, timeout=600)
    out = r.stdout + r.stderr
    assert "AddressSanitizer" not in out and "runtime error" not in out, out[-4000:]
    assert r.returncode == 0, out[-4000:]
    return r.stdout


def _mutants(rng, good, n, span):
    out = []
    for k in range(n):
        b = bytearray(good)
        kind = k % 4
        if kind == 0:                       # truncate anywhere
            b = b[:int(rng.integers(0, len(b)))]
        elif kind == 1:                     # random bytes in the header / index
            for _ in range(int(rng.integers(1, 5))):
                b[int(rng.integers(0, span))] = int(rng.integers(0, 256))
        elif kind == 2:                     # a random 32- or 64-bit field value
            w = 4 if rng.integers(0, 2) == 0 else 8
            pos = int(rng.integers(0, (span - w) // 4)) * 4
            v = int(rng.choice([0, 1, 0xFFFFFFFF, 1 << 31, int(rng.integers(0, 1 << 30))]))
            b[pos:pos + w] = (v & ((1 << (8 * w)) - 1)).to_bytes(w, "little")
        else:                               # flip one bit anywhere
            pos = int(rng.integers(0, len(b)))
            b[pos] ^= 1 << int(rng.integers(0, 8))
        out.append(bytes(b))
    return out


def test_reader_and_writer_under_sanitizers(asan_bin, tmp_path):
    rng = np.random.default_rng(11)
    good = tmp_path / "good.ssm"
    py_write(good, {}, small_tensors(rng))
    files, expect = [str(good)], {}
    gb = open(good, "rb").read()
    for name, mutate, msg in CASES:
        p = tmp_path / f"case_{re.sub(r'[^a-z0-9]', '_', name)}.ssm"
        open(p, "wb").write(bytes(mutate(bytearray(gb))))
        files.append(str(p))
        expect[str(p)] = msg.replace("SSMFile: ", "")
    data_off = int.from_bytes(gb[24:32], "little")
    for i, m in enumerate(_mutants(rng, gb, 300, data_off)):
        p = tmp_path / f"mut_{i}.ssm"
        open(p, "wb").write(m)
        files.append(str(p))
    model = tmp_path / "model.ssm"
    out = _run(asan_bin, ["--write", str(model), *files])
    lines = {ln.split("\t")[0].split(" ")[1]: ln for ln in out.splitlines() if ln}
    assert lines[str(model)].startswith("opened ")
    assert lines[str(good)].startswith("opened ")
    for p, msg in expect.items():
        assert lines[p].startswith("rejected ") and msg in lines[p], lines[p]
    assert len(lines) == len(files) + 1
    # mutants of the writer-made model (its index has 20 entries)
    mb = open(model, "rb").read()
    moff = int.from_bytes(mb[24:32], "little")
    files2 = []
    for i, m in enumerate(_mutants(rng, mb, 200, moff)):
        p = tmp_path / f"mmut_{i}.ssm"
        open(p, "wb").write(m)
        files2.append(str(p))
    out2 = _run(asan_bin, files2)
    assert len([ln for ln in out2.splitlines() if ln]) == len(files2)

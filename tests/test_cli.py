"""lssm_cli, the Linux counterpart of the reference's apps/lite_ssm_cli.cpp, on
the CPU: flag errors with the reference's messages and exit codes
(lite_ssm_cli.cpp:68-71, 106-147), --probe-only's report with RSS from
/proc/self/statm (:161-167, 180-211), and the text front end's tokenizer
check (:215-221).  Nothing here touches a GPU: --probe-only maps the file and
reads its index only."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLI = os.path.join(ROOT, "lite_ssm_amd", "lssm_cli")

pytestmark = pytest.mark.skipif(not os.path.exists(CLI), reason="lssm_cli not built")


def run(*args):
    return subprocess.run([CLI, *args], capture_output=True, text=True, timeout=60)


@pytest.mark.parametrize("args,msg", [
    (["--bogus"], "unknown flag: --bogus"),
    ([], "provide a prompt text positionally, --input-ids, or --probe-only"),
    (["--input-ids", "1,2", "hello"], "can't combine --input-ids with a positional prompt"),
    (["--tokens"], "--tokens expects an argument"),
    (["hello", "world"], "text prompts need SentencePiece"),
])
def test_flag_errors(args, msg):
    r = run(*args)
    assert r.returncode == 2, r
    assert f"lite-ssm: {msg}" in r.stderr


def test_help_exits_zero():
    r = run("--help")
    assert r.returncode == 0 and "--input-ids" in r.stderr and "--probe-only" in r.stderr


def test_missing_model_is_a_library_error(tmp_path):
    r = run("--model", str(tmp_path / "absent.ssm"), "--probe-only")
    assert r.returncode == 1 and r.stderr.startswith("lite-ssm: open: ")


def test_probe_only_report(tmp_path):
    from lite_ssm_amd import ssm as S
    from lite_ssm_amd.model import shape
    import oracle as O
    p = tmp_path / "m.ssm"
    sh = shape("mamba2-130m", n_layer=2, vocab_size=1024)
    S.write_random(p, sh, O.F16, O.W_Q8_G32, seed=1)
    with S.SSMFile(p) as f:
        n = len(f)
    r = run("--model", str(p), "--probe-only")
    assert r.returncode == 0, r.stderr
    lines = r.stdout.splitlines()
    assert lines[0] == "== probe-only mmap stress =="
    assert f"tensors indexed   : {n}" in r.stdout
    size_gb = os.path.getsize(p) / 1e9
    assert f"({size_gb:.2f} GB)" in r.stdout
    # every page of the file touched: the resident set grew by about the file
    rss = {l.split(":")[0].strip(): float(l.split(":")[1].split("MB")[0]) for l in lines[1:]
           if "rss" in l}
    assert rss["rss after scan"] - rss["rss after mmap"] >= 0.9 * os.path.getsize(p) / 2**20


def test_text_front_end_needs_tokenizer(tmp_path):
    r = subprocess.run([sys.executable, "-m", "lite_ssm_amd.cli", "--tokenizer", str(tmp_path / "t.model"),
                        "hello"], capture_output=True, text=True, cwd=ROOT, timeout=120)
    assert r.returncode != 0
    assert f"SentencePiece model not found at '{tmp_path / 't.model'}'" in r.stderr


def test_text_front_end_passes_id_mode_through():
    r = subprocess.run([sys.executable, "-m", "lite_ssm_amd.cli", "--bogus"], capture_output=True, text=True,
                       cwd=ROOT, timeout=120)
    assert r.returncode == 2 and "unknown flag: --bogus" in r.stderr

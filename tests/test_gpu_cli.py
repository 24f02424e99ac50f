"""lssm_cli on the GPU: the ids it prints and the logits it dumps equal the
engine's own greedy run on the same file (apps/lite_ssm_cli.cpp:296-346 decode
loop, --dump-logits and id output), --top-p draws what sampler.cpp:39-79 draws
from the dumped logits, --eos stops after the EOS id, an id past the vocabulary
is rejected with the reference's message (:238-240), and the Python text front
end round-trips a prompt through a SentencePiece model trained here."""
import os
import struct
import subprocess
import sys

import numpy as np
import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLI = os.path.join(ROOT, "lite_ssm_amd", "lssm_cli")
VOCAB = 2048
PROMPT = [5, 77, 1023, 9, 2047, 0, 314, 15, 92, 600, 11]


@pytest.fixture(scope="module")
def model_file(tmp_path_factory):
    from lite_ssm_amd import ssm as S
    from lite_ssm_amd.model import shape
    p = tmp_path_factory.mktemp("cli") / "m.ssm"
    S.write_random(p, shape("mamba2-130m", n_layer=2, vocab_size=VOCAB), O.BF16, O.W_Q4_G64, seed=4)
    return p


def run(*args):
    print("case: lssm_cli", " ".join(map(str, args))[:160], flush=True)
    return subprocess.run([CLI, *map(str, args)], capture_output=True, text=True, timeout=120)


def engine_greedy(ctx, path, prompt, steps):
    """Greedy ids and last logits (fp32) of the engine on the same file."""
    from lite_ssm_amd import ssm as S
    from lite_ssm_amd.model import Engine
    with S.SSMFile(path) as f:
        fm = f.model(ctx)
        eng = Engine(ctx, fm, 1, max(len(prompt), fm.shape.chunk_size))   # the CLI's max_seq
        try:
            nxt = torch.zeros(1, dtype=torch.int32, device="cuda")
            eng.prefill(torch.tensor([prompt], dtype=torch.int32).cuda(), nxt)
            out = [int(nxt.item())]
            for _ in range(steps - 1):
                eng.decode(nxt.clone(), nxt)
                out.append(int(nxt.item()))
            return out, eng.logits(1).float().cpu().numpy()[0]
        finally:
            eng.close()


def top_p_pick(logits, top_p, temperature, seed):
    """sampler.cpp:39-79 in float32, sums in order."""
    f = np.float32
    t = f(temperature) if temperature > 1e-6 else f(1.0)
    order = sorted(range(len(logits)), key=lambda i: -logits[i])   # stable: ties by index
    top = f(logits[order[0]]) / t
    p = [np.exp(f(logits[i]) / t - top, dtype=np.float32) for i in order]
    total = f(0.0)
    for v in p:
        total = f(total + v)
    p = [f(v / total) for v in p]
    keep, run_ = len(p), f(0.0)
    for i, v in enumerate(p):
        run_ = f(run_ + v)
        if run_ >= f(top_p):
            keep = i + 1
            break
    mass = f(0.0)
    for v in p[:keep]:
        mass = f(mass + v)
    s = seed if seed else 1
    m = (1 << 64) - 1
    s ^= (s << 13) & m
    s ^= s >> 7
    s ^= (s << 17) & m
    r = f(f(s >> 40) / f(1 << 24)) * mass
    acc = f(0.0)
    for i in range(keep):
        acc = f(acc + p[i])
        if r <= acc:
            return order[i]
    return order[keep - 1]


def test_cli_greedy_matches_engine(ctx, model_file, tmp_path):
    dump = tmp_path / "logits.bin"
    r = run("--model", model_file, "--input-ids", ",".join(map(str, PROMPT)), "--tokens", 12,
            "--dump-logits", dump)
    assert r.returncode == 0, r.stderr
    ids = [int(v) for v in r.stdout.strip().split(",")]
    assert "[lite-ssm] prefill" in r.stderr and "generated=12" in r.stderr
    want, logits = engine_greedy(ctx, model_file, PROMPT, 12)
    assert ids == want
    got = np.fromfile(dump, dtype=np.float32)
    assert got.shape == (VOCAB,)
    assert np.array_equal(got, logits)          # same kernels, same inputs: bit-identical
    assert int(np.argmax(got)) == ids[-1]


def test_cli_eos_stops(ctx, model_file):
    want, _ = engine_greedy(ctx, model_file, PROMPT, 6)
    r = run("--model", model_file, "--input-ids", ",".join(map(str, PROMPT)), "--tokens", 50,
            "--eos", want[2], "--quiet")
    assert r.returncode == 0 and r.stderr == ""
    ids = [int(v) for v in r.stdout.strip().split(",")]
    stop = want.index(want[2]) + 1               # first occurrence ends the loop
    assert ids == want[:stop]


@pytest.mark.parametrize("top_p,temp,seed", [(0.9, 1.0, 0xCAFEBABE), (0.5, 0.7, 7), (1e-6, 1.0, 3)])
def test_cli_top_p_first_draw(model_file, tmp_path, top_p, temp, seed):
    dump = tmp_path / "l.bin"
    r = run("--model", model_file, "--input-ids", ",".join(map(str, PROMPT)), "--tokens", 1,
            "--top-p", top_p, "--temperature", temp, "--seed", seed, "--dump-logits", dump, "--quiet")
    assert r.returncode == 0, r.stderr
    logits = np.fromfile(dump, dtype=np.float32)
    got, want = int(r.stdout.strip()), top_p_pick(logits, top_p, temp, seed)
    # std::sort leaves the order of equal logits open: the draw lands on the
    # same position of the sorted list, which may hold another index of the
    # same logit
    assert logits[got] == logits[want], (got, want)
    if top_p < 1e-3:                              # nucleus of one: the argmax
        assert int(r.stdout.strip()) == int(np.argmax(logits))


def test_cli_rejects_out_of_vocab(model_file):
    r = run("--model", model_file, "--input-ids", f"1,{VOCAB}", "--tokens", 2)
    assert r.returncode == 2 and f"lite-ssm: input id {VOCAB} out of vocab range" in r.stderr


def test_text_front_end_round_trip(ctx, tmp_path):
    import sentencepiece as spm
    from lite_ssm_amd import ssm as S
    from lite_ssm_amd.model import shape
    model_file = tmp_path / "m64.ssm"             # vocabulary of the tokenizer below
    S.write_random(model_file, shape("mamba2-130m", n_layer=2, vocab_size=64), O.BF16, O.W_Q4_G64, seed=5)
    corpus = tmp_path / "c.txt"
    words = ["state", "space", "model", "scan", "chunk", "decode", "prefill", "token", "layer", "head"]
    rng = np.random.default_rng(0)
    corpus.write_text("\n".join(" ".join(rng.choice(words, 8)) for _ in range(400)))
    prefix = str(tmp_path / "tok")
    spm.SentencePieceTrainer.train(input=str(corpus), model_prefix=prefix, vocab_size=64,
                                   model_type="bpe", minloglevel=2)
    sp = spm.SentencePieceProcessor(model_file=prefix + ".model")
    text = "state space model decode"
    ids = sp.encode(text)
    want, _ = engine_greedy(ctx, model_file, ids, 5)
    print("case: python -m lite_ssm_amd.cli text mode", flush=True)
    r = subprocess.run([sys.executable, "-m", "lite_ssm_amd.cli", "--model", str(model_file), "--tokenizer",
                        prefix + ".model", "--tokens", "5", "--eos", "999999", "--quiet", *text.split()],
                       capture_output=True, text=True, cwd=ROOT, timeout=120)
    assert r.returncode == 0, r.stderr
    assert r.stdout == text + sp.decode(want) + "\n"
    # a model whose ids the tokenizer cannot decode is refused with a message
    print("case: text mode, model vocabulary larger than the tokenizer's", flush=True)
    big = tmp_path / "m2048.ssm"
    S.write_random(big, shape("mamba2-130m", n_layer=2, vocab_size=2048), O.BF16, O.W_Q4_G64, seed=5)
    r = subprocess.run([sys.executable, "-m", "lite_ssm_amd.cli", "--model", str(big), "--tokenizer",
                        prefix + ".model", "--tokens", "40", "--quiet", *text.split()],
                       capture_output=True, text=True, cwd=ROOT, timeout=120)
    if r.returncode != 0:
        assert "outside the tokenizer's 64 pieces" in r.stderr

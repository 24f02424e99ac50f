"""Text front end of ``lssm_cli``: ``python -m lite_ssm_amd.cli [flags] "prompt"``.

The reference CLI tokenizes text prompts with SentencePiece linked into the
binary (apps/lite_ssm_cli.cpp:215-231) and streams the decoded continuation
(:271-294).  SentencePiece's C++ library is not part of this build, but its
Python module is, so this wrapper encodes the prompt with the ``--tokenizer``
model, runs ``lssm_cli`` with ``--input-ids`` and the remaining flags, and
prints the prompt followed by the decoded continuation once generation ends
(whole-sequence decode, so word-boundary markers and byte pieces come out as
the reference's streaming produces them).  The EOS id defaults to the
tokenizer's, as in the reference (:250-252).  Without a positional prompt it
hands every flag to ``lssm_cli`` unchanged.
"""
from __future__ import annotations

import os
import subprocess
import sys

CLI_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lssm_cli")
# flags of lssm_cli that take a value (the others are switches)
_VALUED = {"--model", "--tokenizer", "--tokens", "--top-p", "--temperature", "--seed", "--input-ids",
           "--dump-logits", "--eos"}


def split_args(argv):
    """(flags with their values, positional words, tokenizer path, eos given)."""
    flags, words, tokenizer, eos_set = [], [], "tokenizer.model", False
    i = 0
    while i < len(argv):
        a = argv[i]
        if a in _VALUED:
            if i + 1 >= len(argv):
                raise SystemExit(f"lite-ssm: {a} expects an argument")
            if a == "--tokenizer":
                tokenizer = argv[i + 1]
            else:
                flags += [a, argv[i + 1]]
                eos_set |= a == "--eos"
            i += 2
            continue
        (flags if a.startswith("-") else words).append(a)
        i += 1
    return flags, words, tokenizer, eos_set


def main(argv=None) -> int:
    argv = list(sys.argv[1:] if argv is None else argv)
    if not os.path.exists(CLI_PATH):
        raise SystemExit(f"lite-ssm: {CLI_PATH} is not built (make -C lite_ssm_amd/csrc)")
    flags, words, tokenizer, eos_set = split_args(argv)
    if not words:
        return subprocess.run([CLI_PATH] + argv).returncode
    if "--input-ids" in flags:
        raise SystemExit("lite-ssm: can't combine --input-ids with a positional prompt")
    if not os.path.exists(tokenizer):
        raise SystemExit(f"lite-ssm: SentencePiece model not found at '{tokenizer}'. "
                         "Generate with: tools/export_tokenizer.py")
    import sentencepiece as spm
    sp = spm.SentencePieceProcessor(model_file=tokenizer)
    text = " ".join(words)
    ids = sp.encode(text)
    if not ids:
        raise SystemExit("lite-ssm: empty prompt after tokenization")
    cmd = [CLI_PATH] + flags + ["--input-ids", ",".join(map(str, ids))]
    if not eos_set and sp.eos_id() >= 0:
        cmd += ["--eos", str(sp.eos_id())]
    r = subprocess.run(cmd, stdout=subprocess.PIPE)
    if r.returncode != 0:
        return r.returncode
    out = r.stdout.decode().strip()
    gen = [int(v) for v in out.split(",")] if out else []
    bad = [v for v in gen if v >= sp.get_piece_size()]
    if bad:
        raise SystemExit(f"lite-ssm: generated id {bad[0]} is outside the tokenizer's "
                         f"{sp.get_piece_size()} pieces (model and tokenizer vocabularies differ)")
    sys.stdout.write(text + sp.decode(gen) + "\n")
    sys.stdout.flush()
    return 0


if __name__ == "__main__":
    sys.exit(main())

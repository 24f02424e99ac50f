""".ssm files through the C ABI (lssm_ssm_*), no GPU: layout, validation, writer,
quantizer, random-init model writer, and the model's weight lookups.

Pins: the reference commits no .ssm files (.gitignore:27-28), but its loader test
fixes the layout of the real mamba2-130m export: 219 tensors, f16, the embedding
first at byte 17600 (tests/test_mmap_loader.cpp:64-92).  The on-disk structures are
checked against a struct-based reader and writer written here from the spec
(include/lite_ssm/ssm_format.hpp), in both directions.  Error messages are the
reference loader's (src/core/ssm_loader.cpp:54-135).  The quantizer is checked
byte for byte against the oracle's and torch's restatements of the exporter.
"""
import re
import struct

import numpy as np
import pytest
import torch

import lite_ssm_amd as L
import oracle as O
from lite_ssm_amd import model as M
from lite_ssm_amd import ssm as S

HDR = struct.Struct("<4sIIIQQ" + "I" * 12 + "4I")          # 96 bytes
ENT = struct.Struct("<IIIIQQ")                              # 32 bytes


def a8(x):
    return (x + 7) // 8 * 8


def a64(x):
    return (x + 63) // 64 * 64


def py_read(path):
    """Independent reader: (header tuple, [(name, dtype, shape, offset, nbytes)])."""
    b = open(path, "rb").read()
    h = HDR.unpack_from(b, 0)
    assert h[0] == b"LSSM" and h[1] == 1 and h[2] == 96
    n, pos = h[3], h[4]
    out = []
    for _ in range(n):
        name_len, rank, dtype, _pad, off, nb = ENT.unpack_from(b, pos)
        shape = struct.unpack_from(f"<{rank}Q", b, pos + 32)
        name = b[pos + 32 + 8 * rank: pos + 32 + 8 * rank + name_len].decode()
        pos += a8(32 + 8 * rank + name_len)
        out.append((name, dtype, shape, off, nb))
    return h, out, b


def py_write(path, hp, tensors, *, version=1, header_size=96, magic=b"LSSM"):
    """Independent writer: tensors = [(name, dtype, shape, bytes)]."""
    index = b""
    offs = []
    data_off = a64(96 + sum(a8(32 + 8 * len(s) + len(n)) for n, _, s, _ in tensors))
    off = data_off
    for n, dt, s, d in tensors:
        offs.append(off)
        off = a64(off + len(d))
    for (n, dt, s, d), o in zip(tensors, offs):
        e = ENT.pack(len(n), len(s), dt, 0, o, len(d)) + struct.pack(f"<{len(s)}Q", *s) + n.encode()
        index += e + b"\0" * (a8(len(e)) - len(e))
    fields = [hp.get(k, 0) for k in S.HEADER_FIELDS]
    head = HDR.pack(magic, version, header_size, len(tensors), 96, data_off, *fields, 0, 0, 0, 0)
    buf = bytearray(head + index)
    buf += b"\0" * (data_off - len(buf))
    for (n, dt, s, d), o in zip(tensors, offs):
        buf += b"\0" * (o - len(buf))
        buf += d
    open(path, "wb").write(bytes(buf))


def small_tensors(rng):
    f16 = rng.standard_normal(24).astype(np.float16)
    q = rng.integers(0, 256, 64 * 4 // 2 + 64 * 4 // 32 * 2, dtype=np.uint8)
    return [("a.weight", 0, (4, 6), f16.tobytes()),
            ("b.bias", 2, (5,), rng.standard_normal(5).astype(np.float32).tobytes()),
            ("proj.weight", 6, (4, 64), q.tobytes()),
            ("conv.weight", 1, (3, 1, 4), rng.integers(0, 65535, 12, dtype=np.uint16).tobytes())]


# --------------------------------------------------------------------------- format rules
def test_packed_nbytes_rule():
    n = 3352 * 768
    assert S.packed_nbytes(S.DTYPE_INT4_B32, n) == n // 2 + n // 32 * 2   # ssm_format.hpp:64-69
    assert S.packed_nbytes(S.DTYPE_Q4_G64, n) == n // 2 + n // 64 * 2
    assert S.packed_nbytes(S.DTYPE_Q8_G32, n) == n + n // 32 * 2
    for dt, size in ((0, 2), (1, 2), (2, 4), (3, 1), (4, 1), (5, 4)):
        assert S.packed_nbytes(dt, 1000) == 1000 * size
    assert S.packed_nbytes(9, 1000) == 0


def test_layout_of_the_reference_130m_export(tmp_path):
    """The 130M tensor set (exporter names, state-dict order, separate lm_head, f16)
    puts the embedding at byte 17600, as the reference's loader test requires."""
    p = tmp_path / "m130.ssm"
    hp = dict(d_model=768, n_layer=24, d_state=128, d_conv=4, expand=2, vocab_size=50288,
              n_heads=24, d_head=64, chunk_size=256, default_dtype=0, n_groups=1)
    w = S.Writer(p, **hp)
    w.declare("backbone.embeddings.weight", 0, (50288, 768))
    for i in range(24):
        pre = f"backbone.layers.{i}."
        for n, s in (("mixer.dt_bias", (24,)), ("mixer.A_log", (24,)), ("mixer.D", (24,)),
                     ("mixer.conv1d.weight", (1792, 1, 4)), ("mixer.conv1d.bias", (1792,)),
                     ("mixer.in_proj.weight", (3352, 768)), ("mixer.norm.weight", (1536,)),
                     ("mixer.out_proj.weight", (768, 1536)), ("norm.weight", (768,))):
            w.declare(pre + n, 0, s)
    w.declare("backbone.norm_f.weight", 0, (768,))
    w.declare("lm_head.weight", 0, (50288, 768))
    w.finish()                      # nothing put: payloads read as zeros (sparse file)
    with S.SSMFile(p) as f:
        c = f.config()
        assert (c["d_model"], c["n_layer"], c["vocab_size"], c["n_heads"], c["d_head"],
                c["chunk_size"], c["default_dtype"]) == (768, 24, 50288, 24, 64, 256, 0)
        assert len(f) == 219
        emb = f.at("backbone.embeddings.weight")
        assert (emb.dtype, emb.rank, emb.shape[0], emb.shape[1]) == (0, 2, 50288, 768)
        assert emb.offset == 17600
        assert emb.nbytes == 50288 * 768 * 2
        ip = f.at("backbone.layers.12.mixer.in_proj.weight")
        assert (ip.rank, ip.shape[0], ip.shape[1]) == (2, 3352, 768)
        assert all(t.offset % 64 == 0 for _, t in f.entries())
    _, ents, _ = py_read(p)
    assert ents[0][3] == 17600 and len(ents) == 219


def test_cpp_writer_matches_independent_reader(tmp_path, rng):
    p = tmp_path / "w.ssm"
    ts = small_tensors(rng)
    hp = dict(d_model=7, n_layer=3, d_state=5, vocab_size=11, n_groups=2, norm_before_gate=1,
              default_dtype=1)
    w = S.Writer(p, **hp)
    for n, dt, s, _ in ts:
        w.declare(n, dt, s)
    for n, dt, s, d in reversed(ts):            # any order
        w.put(n, np.frombuffer(d, np.uint8))
    w.finish()
    h, ents, b = py_read(p)
    assert h[3] == len(ts) and h[4] == 96 and h[5] % 64 == 0
    assert list(h[6:18]) == [hp.get(k, 0) for k in S.HEADER_FIELDS]
    for (n, dt, s, d), (n2, dt2, s2, off, nb) in zip(ts, ents):
        assert (n, dt, s, len(d)) == (n2, dt2, s2, nb)
        assert off % 64 == 0 and b[off:off + nb] == d
    assert len(b) == ents[-1][3] + ents[-1][4]


def test_independent_writer_matches_cpp_reader(tmp_path, rng):
    p = tmp_path / "py.ssm"
    ts = small_tensors(rng)
    py_write(p, dict(d_model=7, n_groups=0), ts)
    with S.SSMFile(p) as f:
        assert f.header.n_groups == 1                         # 0 reads as 1 (ssm_loader.cpp:40)
        assert f.names() == [t[0] for t in ts]
        for n, dt, s, d in ts:
            t = f.at(n)
            assert (t.dtype, t.rank, tuple(t.shape[:t.rank])) == (dt, len(s), s)
            assert f.raw(n).tobytes() == d
        assert f.find("missing") is None
        with pytest.raises(L.LssmError, match="SSMFile: no tensor named 'missing'"):
            f.at("missing")
        packed, scales = f.array("proj.weight")
        assert packed.shape == (4, 32) and scales.shape == (4, 2)
        assert np.array_equal(f.array("a.weight"), np.frombuffer(ts[0][3], np.uint16).reshape(4, 6))


# --------------------------------------------------------------------------- validation
def _corrupt(tmp_path, rng, mutate, name="bad.ssm"):
    p = tmp_path / "good.ssm"
    py_write(p, {}, small_tensors(rng))
    b = bytearray(open(p, "rb").read())
    b = mutate(b)
    q = tmp_path / name
    open(q, "wb").write(bytes(b))
    return q


def _entry_pos(b, i):
    pos = 96
    for _ in range(i):
        name_len, rank = struct.unpack_from("<II", b, pos)
        pos += a8(32 + 8 * rank + name_len)
    return pos


def _set(fmt, off, v):
    def f(b):
        struct.pack_into(fmt, b, off, v)
        return b
    return f


def _set_entry(i, field_off, fmt, v):
    def f(b):
        struct.pack_into(fmt, b, _entry_pos(b, i) + field_off, v)
        return b
    return f


def _dup_name(b):
    # rename tensor 1 ("b.bias", 6 bytes) to "a.weig" is not equal; make tensor 0's
    # name equal tensor 1's by writing the same 6 bytes and length
    p0, p1 = _entry_pos(b, 0), _entry_pos(b, 1)
    n1, r1 = struct.unpack_from("<II", b, p1)
    name1 = bytes(b[p1 + 32 + 8 * r1: p1 + 32 + 8 * r1 + n1])
    n0, r0 = struct.unpack_from("<II", b, p0)
    struct.pack_into("<I", b, p0, n1)
    b[p0 + 32 + 8 * r0: p0 + 32 + 8 * r0 + n1] = name1      # n1 <= n0's padded room here
    return b


CASES = [
    ("too small", lambda b: b[:95], "file too small to contain a header (95 bytes)"),
    ("magic", _set("<4s", 0, b"LSSX"), "bad magic; not a .ssm file"),
    ("version", _set("<I", 4, 2), "unsupported version 2 (expected 1)"),
    ("header size", _set("<I", 8, 95), "header_size mismatch"),
    ("index offset", _set("<Q", 16, 64), "index/data offsets out of range"),
    ("data offset", _set("<Q", 24, 1 << 40), "index/data offsets out of range"),
    ("rank 0", _set_entry(1, 4, "<I", 0), "tensor 1 has unsupported rank 0"),
    ("rank 5", _set_entry(2, 4, "<I", 5), "tensor 2 has unsupported rank 5"),
    ("payload", _set_entry(0, 16, "<Q", 1 << 40), "payload for 'a.weight' overflows file"),
    ("nbytes", _set_entry(0, 24, "<Q", 46), "'a.weight' nbytes=46 but expected packed=48"),
    ("dtype", _set_entry(2, 8, "<I", 7), "'proj.weight' nbytes=144 but expected packed=136"),
    ("count", _set("<I", 12, 40), "SSMFile: "),
    ("name", _set_entry(3, 0, "<I", 1 << 30), "out-of-bounds read while parsing tensor name"),
    ("overran", _set("<Q", 24, 128), "index walk overran data_offset"),
    ("duplicate", _dup_name, "duplicate tensor name in index"),
]


@pytest.mark.parametrize("case,mutate,msg", CASES, ids=[c[0] for c in CASES])
def test_loader_rejects_bad_files(tmp_path, rng, case, mutate, msg):
    q = _corrupt(tmp_path, rng, mutate)
    with pytest.raises(L.LssmError, match="SSMFile: .*" + re.escape(msg.replace("SSMFile: ", ""))) as ei:
        S.SSMFile(q)
    assert ei.value.code == 1


def test_loader_missing_file(tmp_path):
    with pytest.raises(L.LssmError, match="open"):
        S.SSMFile(tmp_path / "nope.ssm")


def test_writer_errors(tmp_path):
    p = tmp_path / "e.ssm"
    w = S.Writer(p, d_model=4)
    with pytest.raises(L.LssmError, match="not a multiple of 64"):
        w.declare("q", S.DTYPE_Q4_G64, (1, 32))
    with pytest.raises(L.LssmError, match="not a multiple of 64"):   # the first error sticks
        w.finish()
    assert not p.exists()                                            # partial file removed

    w = S.Writer(p, d_model=4)
    w.declare("x", S.DTYPE_F32, (4,))
    with pytest.raises(L.LssmError, match="duplicate tensor name 'x'"):
        w.declare("x", S.DTYPE_F32, (4,))
    with pytest.raises(L.LssmError):
        w.finish()

    w = S.Writer(p, d_model=4)
    w.declare("x", S.DTYPE_F32, (4,))
    with pytest.raises(L.LssmError, match="16 bytes|declared size 16"):
        w.put("x", np.zeros(3, np.float32))
    with pytest.raises(L.LssmError):
        w.finish()

    w = S.Writer(p, d_model=4)
    w.declare("x", S.DTYPE_F32, (4,))
    w.put("x", np.arange(4, dtype=np.float32))
    with pytest.raises(L.LssmError, match="index already written"):
        w.declare("y", S.DTYPE_F32, (4,))
    with pytest.raises(L.LssmError):
        w.finish()

    w = S.Writer(p, d_model=4)
    w.declare("x", S.DTYPE_F32, (2, 2))
    w.put("x", np.arange(4, dtype=np.float32))
    w.finish()
    with S.SSMFile(p) as f:
        assert np.array_equal(f.array("x"), np.arange(4, dtype=np.float32).reshape(2, 2))


# --------------------------------------------------------------------------- quantizer
@pytest.mark.parametrize("wfmt", [L.W_Q4_B32, L.W_Q4_G64, L.W_Q8_G32])
def test_quantize_matches_oracle_and_torch(rng, wfmt):
    N, K = 37, 256
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float16).astype(np.float32)
    G = M.GROUP[wfmt]
    w[3, :G] = 0.0                                   # all-zero group: scale clamps at 1e-12
    qmax = 127.0 if wfmt == L.W_Q8_G32 else 7.0
    w[5, :G] = np.arange(G) - G / 2                  # integer multiples of the scale
    w[6, :G] = (np.arange(G) % 4 - 1.5) * (3.0 / qmax)  # exact .5 ties at scale 1/ (qmax/3)
    w[6, 0] = 3.0
    packed, scales = S.quantize(w, wfmt)
    op, os_ = O.quantize(w, wfmt)
    assert np.array_equal(packed.reshape(-1), np.asarray(op).reshape(-1).view(np.uint8))
    assert np.array_equal(scales.reshape(-1), np.asarray(os_).reshape(-1).view(np.uint16))
    tp, ts = M.quantize(torch.from_numpy(w), wfmt)
    assert np.array_equal(packed, tp.numpy())
    assert np.array_equal(scales, ts.view(torch.int16).numpy().view(np.uint16))


# --------------------------------------------------------------------------- random model
@pytest.mark.parametrize("act,wfmt", [(L.BF16, L.W_Q4_G64), (L.F16, L.W_Q8_G32),
                                      (L.F16, L.W_Q4_B32), (L.BF16, L.W_DENSE)])
def test_write_random_model(tmp_path, act, wfmt):
    sh = M.shape("mamba2-130m", n_layer=2, vocab_size=512)
    p, p2, p3 = tmp_path / "a.ssm", tmp_path / "b.ssm", tmp_path / "c.ssm"
    S.write_random(p, sh, act, wfmt, seed=7)
    S.write_random(p2, sh, act, wfmt, seed=7)
    S.write_random(p3, sh, act, wfmt, seed=8)
    assert open(p, "rb").read() == open(p2, "rb").read()
    assert open(p, "rb").read() != open(p3, "rb").read()
    with S.SSMFile(p) as f:
        assert len(f) == 1 + 9 * sh.n_layer + 1 and f.find("lm_head.weight") is None
        assert f.header.default_dtype == act
        fm = S.FileModel(f, 1 << 20)                 # any base: checks and offsets only
        assert (fm.act, fm.wfmt) == (act, wfmt)
        assert fm.lm_head == fm.embed == (1 << 20) + f.at("backbone.embeddings.weight").offset
        Lw = fm.layer_structs()[1]
        ip = f.at("backbone.layers.1.mixer.in_proj.weight")
        assert Lw.in_proj_w == (1 << 20) + ip.offset
        if wfmt != L.W_DENSE:
            per = 1 if wfmt == L.W_Q8_G32 else 2
            assert Lw.in_proj_s - Lw.in_proj_w == sh.proj * sh.d_model // per
        host = fm.to_host()
        f32 = lambda a: O.from_act(a, act)  # noqa: E731
        Ly = host["layers"][0]
        dt = np.log1p(np.exp(f32(Ly["dt_bias"]).astype(np.float64)))
        assert dt.min() > 0.99e-3 and dt.max() < 0.101
        A = f32(Ly["A_log"])
        assert A.min() >= 0 and A.max() <= np.log(16.0) + 1e-2
        nw = f32(host["norm_f"])
        assert abs(nw.mean() - 1.0) < 0.03 and 0.07 < nw.std() < 0.13
        cw = f32(Ly["conv1d_w"])
        assert cw.shape == (sh.xbc, sh.d_conv) and 0.28 < cw.std() < 0.32
        if wfmt == L.W_DENSE:
            wi = f32(Ly["in_proj_w"])
        else:
            wi = O.dequant(Ly["in_proj_w"], Ly["in_proj_s"], sh.proj, sh.d_model, wfmt)
        assert 0.018 < np.asarray(wi).std() < 0.022


def test_model_lookup_errors(tmp_path):
    sh = M.shape("mamba2-130m", n_layer=2, vocab_size=512)
    p = tmp_path / "m.ssm"
    S.write_random(p, sh, L.BF16, L.W_Q4_G64, seed=1)
    with S.SSMFile(p) as f:
        with pytest.raises(L.LssmError, match="missing buffer"):
            S.FileModel(f, 0)
    good = open(p, "rb").read()

    def rewrite(drop=None, rename=None, hp=None, retype=None):
        with S.SSMFile(p) as f:
            ents = f.entries()
            out = []
            for n, t in ents:
                if n == drop:
                    continue
                d = f.raw(n).tobytes()
                dt, shape = t.dtype, tuple(t.shape[:t.rank])
                if retype and n == retype[0]:
                    dt, d = retype[1], np.frombuffer(d, np.uint16).astype(np.float32).tobytes()
                out.append((rename.get(n, n) if rename else n, dt, shape, d))
            h = f.config()
        h.update(hp or {})
        q = tmp_path / "x.ssm"
        py_write(q, h, out)
        return q

    def err(q, msg):
        with S.SSMFile(q) as f:
            with pytest.raises(L.LssmError, match=msg):
                S.FileModel(f, 1 << 20)

    err(rewrite(drop="backbone.layers.1.mixer.D"),
        "Mamba2Model: missing tensor 'backbone.layers.1.mixer.D'")
    err(rewrite(hp={"n_heads": 25}), r"n_heads \* d_head")
    err(rewrite(hp={"d_state": 64}), r"in_proj output dim mismatch vs config \(got 3352, expected 3224\)")
    err(rewrite(retype=("backbone.layers.0.mixer.A_log", S.DTYPE_F32)), "'backbone.layers.0.mixer.A_log' has dtype 2")
    err(rewrite(hp={"vocab_size": 513}), "embeddings.weight must be")
    err(rewrite(hp={"n_layer": 3}), "missing tensor 'backbone.layers.2.norm.weight'")
    assert open(p, "rb").read() == good

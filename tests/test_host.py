"""Host-side logic on the CPU: checkpoint format, deterministic synthetic
checkpoints, tokenizer/sampler behaviour, runner flag and error handling,
and the C-ABI library's exported surface (loaded, never called on a GPU)."""
import ctypes as C
import os
import re
import subprocess

import numpy as np
import pytest

from conftest import REPO
from llama2q import BUILD_DIR, GPU_LIB, RUNNER, abi, host


# ---------------------------------------------------------------- format

@pytest.mark.parametrize("bits,group,version,hbytes", [(8, 32, 1, 36), (4, 32, 2, 36), (4, 64, 3, 40),
                                                         (8, 64, 3, 40)])
def test_header_round_trip(bits, group, version, hbytes):
    cfg = host.make_config(64, 128, 2, 4, 2, 300, 16)
    ck = host.synth_checkpoint(cfg, bits, group, seed=1)
    magic, ver = np.frombuffer(ck.data[:8].tobytes(), dtype=np.uint32)
    assert magic == (0x344C4C51 if bits == 4 else 0x384C4C51) and ver == version
    assert np.frombuffer(ck.data[8:36].tobytes(), dtype=np.int32)[5] == -300    # unshared classifier
    h = ck.header
    assert (h.wbits, h.group, h.header_bytes, h.shared_weights) == (bits, group, hbytes, 0)
    assert h.cfg.as_list() == cfg.as_list()
    assert ck.data.nbytes == hbytes + ck.layout().total


def test_layout_matches_reference_tensor_walk():
    """Tensor sizes of runq.c:235-252 (biased u8 / packed nibbles + scales)."""
    cfg = host.make_config(288, 768, 6, 6, 6, 32000, 256)
    d, h, L, V = 288, 768, 6, 32000
    for bits in (8, 4):
        lay = host.layout(cfg, bits, 32)
        qb = lambda r, c: r * c * bits // 8 + r * (c // 32) * 4
        assert lay.rms_att == V * d * 4
        assert lay.wq == lay.rms_att + L * d * 4
        assert lay.wk == lay.wq + qb(L * d, d)
        assert lay.rms_ffn == lay.wo + qb(L * d, d)
        assert lay.w2 == lay.w1 + qb(L * h, d)
        assert lay.rms_final == lay.w3 + qb(L * h, d)
        assert lay.wcls == lay.rms_final + d * 4
        assert lay.total == lay.wcls + qb(V, d)


def test_header_rejects_bad_files():
    buf = np.zeros(64, dtype=np.uint8)
    with pytest.raises(ValueError, match="bad magic"):
        host.parse_header(buf)
    buf[:4] = np.frombuffer(np.uint32(0x384C4C51).tobytes(), dtype=np.uint8)
    buf[4:8] = np.frombuffer(np.uint32(2).tobytes(), dtype=np.uint8)     # QLL8 needs version 1
    with pytest.raises(ValueError, match="bad magic"):
        host.parse_header(buf)
    with pytest.raises(ValueError, match="truncated"):
        host.parse_header(buf[:20])


def test_synth_is_deterministic_and_gaussian():
    cfg = host.make_config(64, 128, 2, 4, 4, 300, 16)
    a = host.synth_checkpoint(cfg, 4, 32, seed=5)
    b = host.synth_checkpoint(cfg, 4, 32, seed=5)
    c = host.synth_checkpoint(cfg, 4, 32, seed=6)
    assert np.array_equal(a.data, b.data) and not np.array_equal(a.data, c.data)
    g = host.gauss(1 << 20, 3, 1, 1.0)
    assert abs(g.mean()) < 5e-3 and abs(g.std() - 1.0) < 5e-3
    assert abs(((g > 1.0).mean()) - 0.1587) < 3e-3
    # element index i of a stream does not depend on how the stream is split
    np.testing.assert_array_equal(host.gauss(100, 3, 1, 1.0, index0=7)[:10], g[7:17])


# ---------------------------------------------------------------- tokenizer / sampler (standalone)

@pytest.fixture()
def tok(tmp_path):
    pieces, scores = host.synth_tokenizer_pieces(32000)
    path = str(tmp_path / "tok.bin")
    host.write_tokenizer(path, pieces, scores)
    t = host.Tokenizer(path, 32000)
    yield t, pieces
    t.close()


def test_tokenizer_encode_decode(tok):
    t, pieces = tok
    ids = t.encode("Once upon a time")
    assert ids[0] == 1                                      # BOS
    assert "".join(pieces[i] for i in ids[1:]) == " Once upon a time"
    assert t.encode("") == [1]
    assert t.encode("", bos=False) == []
    assert t.encode("hi", eos=True)[-1] == 2
    ids = t.encode("é", bos=False)                         # not in the vocab: byte fallback (+3)
    assert ids[1:] == [0xC3 + 3, 0xA9 + 3]
    assert t.decode(1, t.lookup(" Once")) == b"Once"        # leading space dropped after BOS
    assert t.decode(5, 3 + 0x41) == b"A"                    # <0x41> -> the raw byte


def test_sampler_argmax_and_rng():
    s = host.Sampler(5, 0.0, 0.9, 1)
    assert s.sample(np.array([1.0, 3.0, 3.0, 2.0, -1.0], dtype=np.float32)) == 1   # first maximum
    # xorshift64* stream (runq.c:642-650) from a known state
    lib = host.lib()
    st = C.c_ulonglong(42)
    got = [lib.sampler_random_f32(C.byref(st)) for _ in range(3)]
    x = 42
    exp = []
    for _ in range(3):
        x ^= x >> 12
        x ^= (x << 25) & 0xFFFFFFFFFFFFFFFF
        x ^= x >> 27
        u = ((x * 0x2545F4914F6CDD1D) & 0xFFFFFFFFFFFFFFFF) >> 32
        exp.append(np.float32((u >> 8) / 16777216.0))
    assert [np.float32(v) for v in got] == exp


def test_sampler_topp_concentrates():
    logits = np.full(1000, -10.0, dtype=np.float32)
    logits[[3, 7]] = [5.0, 5.2]
    s = host.Sampler(1000, 1.0, 0.5, 7)
    assert {s.sample(logits) for _ in range(50)} <= {3, 7}


# ---------------------------------------------------------------- runner CLI (errors before any GPU work)

def run(*args):
    return subprocess.run([RUNNER, *args], capture_output=True, text=True, timeout=60)


def test_runner_usage_errors():
    r = run()
    assert r.returncode == 1 and "Usage:" in r.stderr
    assert run("m.bin", "-t").returncode == 1              # flag without value
    assert run("m.bin", "-tt", "1").returncode == 1        # flags are exactly two characters
    assert run("m.bin", "-q", "1").returncode == 1         # unknown flag


def test_runner_bad_checkpoint(tmp_path):
    r = run(str(tmp_path / "missing.bin"))
    assert r.returncode == 1 and "Couldn't open file" in r.stderr
    bad = tmp_path / "bad.bin"
    bad.write_bytes(b"\0" * 64)
    r = run(str(bad))
    assert r.returncode == 1 and "bad magic" in r.stderr


# ---------------------------------------------------------------- C ABI surface

def declared_functions(path):
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(l2q_\w+)\s*\(", text)))


def test_gpu_library_exports_every_declared_symbol():
    names = declared_functions(os.path.join(REPO, "include", "l2q.h"))
    assert "l2q_engine_forward" in names and "l2q_gemv_q4" in names
    lib = C.CDLL(GPU_LIB)
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert set(names) <= set(abi.SIGNATURES), set(names) - set(abi.SIGNATURES)


def test_abi_constants_equal_the_header_defines():
    """Every L2Q_* integer the Python binding names equals the header's."""
    text = open(os.path.join(REPO, "include", "l2q.h")).read()
    defines = {k: int(v) for k, v in re.findall(r"#define\s+(L2Q_\w+)\s+(-?\d+)", text)}
    names = [n for n in dir(abi) if n.startswith("L2Q_") and isinstance(getattr(abi, n), int)]
    assert len(names) >= 10
    for n in names:
        assert n in defines, n
        assert getattr(abi, n) == defines[n], n


def test_missing_library_fails_loudly(monkeypatch):
    monkeypatch.setattr(abi, "_lib", None)
    monkeypatch.setattr(abi, "GPU_LIB", os.path.join(BUILD_DIR, "nonexistent.so"))
    with pytest.raises(RuntimeError, match="not built"):
        abi.lib()

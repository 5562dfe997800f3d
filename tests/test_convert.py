"""llama2q_convert: llama2.c v0 fp32 checkpoint -> QLL8 / QLL4.

The input is a small fp32 checkpoint in the v0 layout (v0-fp32/run.c:111-162:
28-byte Config, tensors in order, two RoPE tables, wcls when vocab < 0).
Checks: the header and every fp32 tensor are copied byte for byte; every
quantized matrix equals the reference tools' closed form
(tools/quantize_int8.py:52-63, tools/quantize_int4.py:38-51) evaluated in
numpy float32; the shared-classifier cases follow the tools (wcls omitted,
vocab sign kept) or, with -u, carry the quantized embedding as wcls; and the
converted QLL8 G32 file runs bit-identically through the compiled reference
runq.c and the oracle.
"""
import os
import struct
import subprocess

import numpy as np
import pytest

from conftest import PKG
from llama2q import host
import oracle_py as O

CONVERT = os.path.join(PKG, "build", "llama2q_convert")
pytestmark = pytest.mark.skipif(not os.path.exists(CONVERT), reason="llama2q_convert not built")

DIM, HID, L, NH, NKV, V, SEQ = 128, 320, 2, 4, 2, 384, 48


def write_v0(path, shared, seed=3):
    """A random llama2.c v0 fp32 checkpoint; returns its tensors."""
    rng = np.random.default_rng(seed)
    hs, kv = DIM // NH, DIM * NKV // NH
    g = lambda *shape: (rng.standard_normal(shape) * 0.02).astype(np.float32)
    t = {
        "emb": g(V, DIM), "rms_att": (1 + g(L, DIM)).astype(np.float32),
        "wq": g(L * DIM, DIM), "wk": g(L * kv, DIM), "wv": g(L * kv, DIM), "wo": g(L * DIM, DIM),
        "rms_ffn": (1 + g(L, DIM)).astype(np.float32),
        "w1": g(L * HID, DIM), "w2": g(L * DIM, HID), "w3": g(L * HID, DIM),
        "rms_final": (1 + g(DIM)).astype(np.float32),
        "rope": g(SEQ * hs),           # the two legacy freq_cis tables, skipped by every reader
        "wcls": g(V, DIM),
    }
    t["wq"][0, :32] = 0.0              # an all-zero group: scale 1e-8
    with open(path, "wb") as f:
        f.write(struct.pack("7i", DIM, HID, L, NH, NKV, V if shared else -V, SEQ))
        for k in ("emb", "rms_att", "wq", "wk", "wv", "wo", "rms_ffn", "w1", "w2", "w3", "rms_final", "rope"):
            f.write(t[k].tobytes())
        if not shared:
            f.write(t["wcls"].tobytes())
    return t


def q8_closed_form(w, group):
    wb = w.reshape(w.shape[0], -1, group)
    scale = (np.abs(wb).max(axis=2) / np.float32(127.0)).astype(np.float32)
    scale[scale == 0.0] = np.float32(1e-8)
    q = np.clip(np.rint(wb / scale[:, :, None]), -127.0, 127.0)
    return (q + 128.0).astype(np.uint8).reshape(w.shape), scale


def q4_closed_form(w, group, div):
    wb = w.reshape(w.shape[0], -1, group)
    scale = (np.abs(wb).max(axis=2) / np.float32(div)).astype(np.float32)
    scale[scale == 0.0] = np.float32(1e-8)
    q = np.clip(np.rint(wb / scale[:, :, None]), -8.0, 7.0)
    qi = (q.astype(np.int16) & 0xF).astype(np.uint8)
    packed = (qi[:, :, 0::2] | (qi[:, :, 1::2] << 4)).astype(np.uint8)
    return packed.reshape(w.shape[0], -1), scale


def run_convert(src, dst, *args):
    r = subprocess.run([CONVERT, src, dst, *args], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return np.fromfile(dst, dtype=np.uint8)


def walk(buf, wbits, group, wcls_present, div=8.0):
    """Yield (name, array) for every tensor of a QLL file, after the header."""
    off = 40 if group != 32 else 36
    kv = DIM * NKV // NH
    shapes = [("emb", (V, DIM), "f"), ("rms_att", (L, DIM), "f"), ("wq", (L * DIM, DIM), "q"),
              ("wk", (L * kv, DIM), "q"), ("wv", (L * kv, DIM), "q"), ("wo", (L * DIM, DIM), "q"),
              ("rms_ffn", (L, DIM), "f"), ("w1", (L * HID, DIM), "q"), ("w2", (L * DIM, HID), "q"),
              ("w3", (L * HID, DIM), "q"), ("rms_final", (DIM,), "f")]
    if wcls_present:
        shapes.append(("wcls", (V, DIM), "q"))
    for name, shape, kind in shapes:
        if kind == "f":
            n = int(np.prod(shape)) * 4
            yield name, buf[off:off + n].view(np.float32).reshape(shape), None
            off += n
        else:
            rows, cols = shape
            nq = rows * cols * wbits // 8
            q = buf[off:off + nq].reshape(rows, cols * wbits // 8)
            off += nq
            ns = rows * (cols // group) * 4
            s = buf[off:off + ns].view(np.float32).reshape(rows, cols // group)
            off += ns
            yield name, q, s
    assert off == buf.size, (off, buf.size)


@pytest.mark.parametrize("wbits,group,div", [(8, 32, None), (8, 64, None), (4, 32, 8.0), (4, 64, 7.0)])
def test_convert_unshared(tmp_path, wbits, group, div):
    src, dst = str(tmp_path / "in.bin"), str(tmp_path / "out.bin")
    t = write_v0(src, shared=False)
    args = ["-b", str(wbits), "-g", str(group)] + (["-d", str(div)] if div else [])
    buf = run_convert(src, dst, *args)
    magic, version = struct.unpack("<2I", buf[:8].tobytes())
    assert magic == (0x384C4C51 if wbits == 8 else 0x344C4C51)
    assert version == (3 if group != 32 else (1 if wbits == 8 else 2))
    assert struct.unpack("<7i", buf[8:36].tobytes()) == (DIM, HID, L, NH, NKV, -V, SEQ)
    if group != 32:
        assert struct.unpack("<I", buf[36:40].tobytes())[0] == group
    for name, q, s in walk(buf, wbits, group, True):
        if s is None:
            np.testing.assert_array_equal(q, t[name], err_msg=name)
            continue
        eq, es = q8_closed_form(t[name], group) if wbits == 8 else q4_closed_form(t[name], group, div)
        np.testing.assert_array_equal(s, es, err_msg=name + " scales")
        np.testing.assert_array_equal(q, eq, err_msg=name)
    # the library's own header parser accepts the file
    h = host.parse_header(buf)
    assert (h.wbits, h.group, h.shared_weights, h.cfg.vocab_size) == (wbits, group, 0, V)


def test_convert_shared_mirrors_tool_and_unshares(tmp_path):
    src = str(tmp_path / "in.bin")
    t = write_v0(src, shared=True)
    buf = run_convert(src, str(tmp_path / "a.bin"))
    assert struct.unpack("<7i", buf[8:36].tobytes())[5] == V     # sign kept, like the tools
    names = [n for n, _, _ in walk(buf, 8, 32, False)]
    assert "wcls" not in names
    buf = run_convert(src, str(tmp_path / "b.bin"), "-u")
    assert struct.unpack("<7i", buf[8:36].tobytes())[5] == -V
    tensors = {n: (q, s) for n, q, s in walk(buf, 8, 32, True)}
    eq, es = q8_closed_form(t["emb"], 32)
    np.testing.assert_array_equal(tensors["wcls"][0], eq)
    np.testing.assert_array_equal(tensors["wcls"][1], es)


def test_convert_rejects_truncated_input(tmp_path):
    src = str(tmp_path / "in.bin")
    write_v0(src, shared=False)
    data = open(src, "rb").read()
    open(src, "wb").write(data[:-100])
    r = subprocess.run([CONVERT, src, str(tmp_path / "o.bin")], capture_output=True, text=True)
    assert r.returncode != 0 and "needs" in r.stderr


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (no reference checkout)")
def test_converted_file_runs_in_reference_runq(tmp_path):
    """The QLL8 G32 output loads in the compiled reference runq.c, whose
    logits equal the oracle's on the same weights, bit for bit."""
    src, dst = str(tmp_path / "in.bin"), str(tmp_path / "out.bin")
    write_v0(src, shared=False, seed=11)
    run_convert(src, dst)
    ck = host.load_checkpoint(dst)
    ref = O.RefRunq(dst)
    orc = O.Oracle(ck.cfg.as_list(), ck.weights, 8, 32)
    token = 5
    for pos in range(8):
        a = ref.forward(token, pos)
        np.testing.assert_array_equal(a, orc.forward(token, pos))
        token = int(np.argmax(a))
    ref.close()

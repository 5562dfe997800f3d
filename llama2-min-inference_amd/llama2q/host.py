"""ctypes binding of build/libl2q_host.so: checkpoint format, deterministic
random-init checkpoints, offline quantizers, tokenizer and sampler."""
import ctypes as C
import os
from dataclasses import dataclass

import numpy as np

from . import HOST_LIB
from .abi import Config

P = C.c_void_p
I = C.c_int
U64 = C.c_uint64
F = C.c_float


class Layout(C.Structure):
    _fields_ = [(n, C.c_size_t) for n in (
        "emb", "rms_att", "wq", "wq_s", "wk", "wk_s", "wv", "wv_s", "wo", "wo_s", "rms_ffn",
        "w1", "w1_s", "w2", "w2_s", "w3", "w3_s", "rms_final", "wcls", "wcls_s", "total")]


class Header(C.Structure):
    _fields_ = [("cfg", Config), ("shared_weights", I), ("wbits", I), ("group", I),
                ("header_bytes", C.c_size_t)]


SIGNATURES = {
    "qll_matrix_bytes": (C.c_size_t, [C.c_size_t, C.c_size_t, I]),
    "qll_layout_compute": (I, [C.POINTER(Config), I, I, C.POINTER(Layout)]),
    "qll_parse_header": (I, [P, C.c_size_t, C.POINTER(Header), C.c_char_p, C.c_size_t]),
    "qll_write_header": (C.c_size_t, [P, C.POINTER(Config), I, I]),
    "qll_quantize_row_q8": (None, [P, I, I, P, P]),
    "qll_quantize_row_q4": (None, [P, I, I, F, P, P]),
    "qll_gauss": (F, [U64, U64, U64]),
    "qll_gauss_fill": (None, [P, C.c_size_t, U64, U64, U64, F]),
    "qll_uniform_int": (I, [U64, U64, U64, I, I]),
    "qll_synth_size": (C.c_size_t, [C.POINTER(Config), I, I]),
    "qll_synth_write": (I, [P, C.POINTER(Config), I, I, F, U64, F]),
    "qll_synth_write_file": (I, [C.c_char_p, C.POINTER(Config), I, I, F, U64, F]),
    "tok_load": (I, [P, C.c_char_p, I, C.c_char_p, I]),
    "tok_free": (None, [P]),
    "tok_lookup": (I, [P, C.c_char_p]),
    "tok_encode": (I, [P, C.c_char_p, I, I, P]),
    "tok_decode": (C.c_char_p, [P, I, I]),
    "tok_write": (I, [C.c_char_p, P, P, I]),
    "sampler_init": (I, [P, I, F, F, C.c_ulonglong]),
    "sampler_free": (None, [P]),
    "sampler_argmax": (I, [P, I]),
    "sampler_softmax": (None, [P, I]),
    "sampler_random_f32": (F, [P]),
    "sampler_sample": (I, [P, P]),
}

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(HOST_LIB):
            raise RuntimeError(f"{HOST_LIB} is not built; run __graft_entry__.build() or make")
        L = C.CDLL(HOST_LIB)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def make_config(dim, hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size, seq_len) -> Config:
    return Config(dim, hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size, seq_len)


# BASELINE configurations (dimensions of the reference's test models).
def config_15m() -> Config:
    """Plumbing model: stories15M shape (dim 288, 6 layers, 6 heads)."""
    return make_config(288, 768, 6, 6, 6, 32000, 256)


def config_7b(seq_len: int = 4096) -> Config:
    """Llama-2-7B shape (dim 4096, 32 layers, 32 heads, hidden 11008)."""
    return make_config(4096, 11008, 32, 32, 32, 32000, seq_len)


def layout(cfg: Config, wbits: int, group: int) -> Layout:
    lay = Layout()
    if lib().qll_layout_compute(C.byref(cfg), wbits, group, C.byref(lay)) != 0:
        raise ValueError("inconsistent config for the checkpoint layout")
    return lay


def parse_header(buf: np.ndarray) -> Header:
    h = Header()
    err = C.create_string_buffer(256)
    rc = lib().qll_parse_header(ptr(buf), buf.nbytes, C.byref(h), err, 256)
    if rc != 0:
        raise ValueError(err.value.decode())
    return h


@dataclass
class Checkpoint:
    """A complete QLL8/QLL4 checkpoint image held in host memory."""
    data: np.ndarray          # uint8, whole file
    header: Header

    @property
    def cfg(self) -> Config:
        return self.header.cfg

    @property
    def wbits(self) -> int:
        return self.header.wbits

    @property
    def group(self) -> int:
        return self.header.group

    @property
    def weights(self) -> np.ndarray:
        """The tensor section (everything after the header)."""
        return self.data[self.header.header_bytes:]

    def layout(self) -> Layout:
        return layout(self.cfg, self.wbits, self.group)

    def save(self, path: str) -> None:
        self.data.tofile(path)


def synth_checkpoint(cfg: Config, wbits: int, group: int, seed: int = 1234, sigma: float = 0.02,
                     q4_divisor: float = 7.0) -> Checkpoint:
    """Random-init checkpoint: N(0, sigma) matrices and embedding, RMSNorm
    weights 1.0, quantized with the offline quantizers (INT4 divisor
    `q4_divisor`: 8 as tools/quantize_int4.py, 7 for the 7B configs)."""
    n = lib().qll_synth_size(C.byref(cfg), wbits, group)
    if n == 0:
        raise ValueError("inconsistent config")
    buf = np.empty(n, dtype=np.uint8)
    if lib().qll_synth_write(ptr(buf), C.byref(cfg), wbits, group, q4_divisor, seed, sigma) != 0:
        raise ValueError("synthetic writer failed")
    return Checkpoint(buf, parse_header(buf))


def load_checkpoint(path: str) -> Checkpoint:
    buf = np.fromfile(path, dtype=np.uint8)
    return Checkpoint(buf, parse_header(buf))


def gauss(n: int, seed: int, stream: int, sigma: float = 1.0, index0: int = 0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().qll_gauss_fill(ptr(out), n, seed, stream, index0, sigma)
    return out


def uniform_ints(n: int, seed: int, stream: int, lo: int, hi: int) -> np.ndarray:
    L = lib()
    return np.array([L.qll_uniform_int(seed, stream, i, lo, hi) for i in range(n)], dtype=np.int32)


def quantize_q8(w: np.ndarray, group: int):
    """Offline INT8 quantizer (tools/quantize_int8.py:52-63): biased u8 + scales."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    q = np.empty((rows, cols), dtype=np.uint8)
    s = np.empty((rows, cols // group), dtype=np.float32)
    L = lib()
    for r in range(rows):
        L.qll_quantize_row_q8(ptr(w[r]), cols, group, ptr(q[r]), ptr(s[r]))
    return q, s


def quantize_q4(w: np.ndarray, group: int, divisor: float = 8.0):
    """Offline INT4 quantizer (tools/quantize_int4.py:38-51): packed nibbles + scales."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    q = np.empty((rows, cols // 2), dtype=np.uint8)
    s = np.empty((rows, cols // group), dtype=np.float32)
    L = lib()
    for r in range(rows):
        L.qll_quantize_row_q4(ptr(w[r]), cols, group, divisor, ptr(q[r]), ptr(s[r]))
    return q, s


def rope_table_bytes(max_t: int, head_size: int) -> int:
    return max_t * head_size * 4


# ---------------------------------------------------------------------------
# tokenizer / sampler


class _TokenizerStruct(C.Structure):
    _fields_ = [("pieces", P), ("scores", P), ("by_text", P), ("vocab_size", I),
                ("max_token_length", C.c_uint), ("byte_text", (C.c_char * 2) * 256)]


class Tokenizer:
    def __init__(self, path: str, vocab_size: int):
        self._t = _TokenizerStruct()
        err = C.create_string_buffer(256)
        if lib().tok_load(C.byref(self._t), path.encode(), vocab_size, err, 256) != 0:
            raise ValueError(err.value.decode())

    def encode(self, text: str, bos: bool = True, eos: bool = False):
        b = text.encode()
        out = np.empty(len(b) + 3, dtype=np.int32)
        n = lib().tok_encode(C.byref(self._t), b, int(bos), int(eos), ptr(out))
        return [int(v) for v in out[:n]]

    def decode(self, prev: int, token: int) -> bytes:
        return lib().tok_decode(C.byref(self._t), prev, token)

    def lookup(self, text: str) -> int:
        return lib().tok_lookup(C.byref(self._t), text.encode())

    def close(self):
        if self._t.pieces:
            lib().tok_free(C.byref(self._t))

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def write_tokenizer(path: str, pieces, scores) -> None:
    n = len(pieces)
    arr = (C.c_char_p * n)(*[p.encode() if isinstance(p, str) else p for p in pieces])
    sc = np.asarray(scores, dtype=np.float32)
    if lib().tok_write(path.encode(), C.cast(arr, P), ptr(sc), n) != 0:
        raise OSError(f"cannot write {path}")


def synth_tokenizer_pieces(vocab_size: int = 32000):
    """Pieces of a synthetic tokenizer.bin for random-id runs: <unk>, BOS,
    EOS, the 256 byte pieces <0xXX>, printable ASCII characters and a few
    words (so prompts encode through the BPE merges), then unique
    placeholder pieces " t<id>"."""
    pieces = ["<unk>", "\n<s>\n", "\n</s>\n"] + [f"<0x{b:02X}>" for b in range(256)]
    scores = [0.0] * len(pieces)
    chars = [chr(c) for c in range(32, 127)]
    pieces += chars
    scores += [-1000.0] * len(chars)
    words = [" O", " On", " Once", " u", " up", " upon", " a", " t", " ti", " tim", " time",
             "nc", "ce", "on", "po", "im", "me", " [", "IN", "ST", "]", " [/", "INST", " [INST]"]
    for i, w in enumerate(words):
        if w not in pieces:
            pieces.append(w)
            scores.append(float(-i))
    while len(pieces) < vocab_size:
        pieces.append(f" t{len(pieces)}")
        scores.append(-2000.0)
    return pieces[:vocab_size], scores[:vocab_size]


class _SamplerStruct(C.Structure):
    _fields_ = [("vocab_size", I), ("temperature", F), ("topp", F),
                ("rng_state", C.c_ulonglong), ("scratch", P)]


class Sampler:
    def __init__(self, vocab_size: int, temperature: float, topp: float, seed: int):
        self._s = _SamplerStruct()
        if lib().sampler_init(C.byref(self._s), vocab_size, temperature, topp, seed) != 0:
            raise MemoryError("sampler")

    def sample(self, logits: np.ndarray) -> int:
        buf = np.ascontiguousarray(logits, dtype=np.float32).copy()
        return lib().sampler_sample(C.byref(self._s), ptr(buf))

    @property
    def rng_state(self) -> int:
        return self._s.rng_state

    def close(self):
        if self._s.scratch:
            lib().sampler_free(C.byref(self._s))
            self._s.scratch = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

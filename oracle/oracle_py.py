"""ctypes binding of the oracle (TEST INFRASTRUCTURE ONLY).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module; the product never does.

* ``Oracle`` binds liboracle.so, the plain-C restatement of the reference
  decode path (oracle.c, each function citing the runq.c lines it follows).
* ``RefRunq`` binds _ref/libref_runq.so, the reference CPU runner
  (v1-int8-vnni/runq.c) compiled unmodified from the reference checkout.
"""
import ctypes as C
import os

import numpy as np

ORACLE_DIR = os.path.dirname(os.path.abspath(__file__))
ORACLE_LIB = os.path.join(ORACLE_DIR, "liboracle.so")
REF_LIB = os.path.join(ORACLE_DIR, "_ref", "libref_runq.so")
REF_BIN = os.path.join(ORACLE_DIR, "_ref", "runq")

P = C.c_void_p
I = C.c_int


def _p(a):
    return None if a is None else a.ctypes.data


_olib = None


def olib():
    global _olib
    if _olib is None:
        L = C.CDLL(ORACLE_LIB)
        sig = {
            "orc_quantize_act": (None, [P, I, I, P, P, P]),
            "orc_matmul_q8": (None, [P, P, P, P, P, P, I, I, I, P]),
            "orc_matmul_q4": (None, [P, P, P, P, P, P, I, I, I, P]),
            "orc_rmsnorm": (None, [P, P, P, I]),
            "orc_softmax": (None, [P, I]),
            "orc_model_create": (P, [P, P, C.c_size_t, I, I, I]),
            "orc_model_free": (None, [P]),
            "orc_forward": (C.POINTER(C.c_float), [P, I, I, P]),
            "orc_greedy": (None, [P, P, I, I, P]),
            "orc_argmax": (I, [P, I]),
            "orc_rope_table": (None, [P, I, I]),
            "orc_rope": (None, [P, P, I, I, I, I]),
            "orc_attention": (None, [P, P, P, P, I, I, I, I, C.c_size_t, C.c_size_t, P, I]),
            "orc_swiglu": (None, [P, P, P, I]),
            "orc_expf_array": (None, [P, P, C.c_size_t]),
            "orc_kv_quant": (None, [P, I, P, P]),
            "orc_attention_kv8": (None, [P, P, P, P, P, P, I, I, I, I] + [C.c_size_t] * 4),
            "orc_model_set_kv8": (I, [P, I]),
            "orc_attention_kv8_ordered": (None, [P, P, P, P, P, P, I, I, I, I] + [C.c_size_t] * 4),
            "orc_attention_kv8_split": (None, [P, P, P, P, P, P, I, I, I, I] + [C.c_size_t] * 4 + [I]),
            "orc_model_set_kv8_splits": (I, [P, I, I]),
        }
        for n, (r, a) in sig.items():
            f = getattr(L, n)
            f.restype = r
            f.argtypes = a
        _olib = L
    return _olib


def argmax(v: np.ndarray) -> int:
    """runq.c:578-585 greedy argmax: the scan from v[0] taking v[i] > max."""
    v = np.ascontiguousarray(v, dtype=np.float32)
    return int(olib().orc_argmax(_p(v), v.size))


def quantize_act(x: np.ndarray, group: int):
    x = np.ascontiguousarray(x, dtype=np.float32)
    n = x.size
    xq = np.empty(n, dtype=np.int8)
    xs = np.empty(n // group, dtype=np.float32)
    xt = np.empty(n // group, dtype=np.float32)
    olib().orc_quantize_act(_p(x), n, group, _p(xq), _p(xs), _p(xt))
    return xq, xs, xt


def matmul(bits: int, xq, xs, xt, w, ws, rows: int, cols: int, group: int, want_dots: bool = True):
    """out[rows] (+ int32 group dots) of the oracle GEMV; w as stored in the
    file (INT8: biased u8 [rows][cols]; INT4: packed [rows][cols/2])."""
    out = np.empty(rows, dtype=np.float32)
    dots = np.empty((rows, cols // group), dtype=np.int32) if want_dots else None
    xq, xs, xt = (np.ascontiguousarray(a) for a in (xq, xs, xt))
    w, ws = np.ascontiguousarray(w), np.ascontiguousarray(ws)
    f = olib().orc_matmul_q4 if bits == 4 else olib().orc_matmul_q8
    f(_p(out), _p(xq), _p(xs), _p(xt), _p(w), _p(ws), rows, cols, group, _p(dots))
    return out, dots


def rmsnorm(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    o = np.empty_like(x)
    olib().orc_rmsnorm(_p(o), _p(x), _p(w), x.size)
    return o


def softmax(x: np.ndarray) -> np.ndarray:
    y = np.ascontiguousarray(x, dtype=np.float32).copy()
    olib().orc_softmax(_p(y), y.size)
    return y


def rope_table(max_t: int, head_size: int) -> np.ndarray:
    t = np.empty(max_t * head_size, dtype=np.float32)
    olib().orc_rope_table(_p(t), max_t, head_size)
    return t


def rope(q: np.ndarray, k: np.ndarray, pos: int, head_size: int):
    """Rotated copies of q [dim] and k [kv_dim] (runq.c:351-365)."""
    q = np.ascontiguousarray(q, dtype=np.float32).copy()
    k = np.ascontiguousarray(k, dtype=np.float32).copy()
    olib().orc_rope(_p(q), _p(k), pos, q.size, k.size, head_size)
    return q, k


def attention(q: np.ndarray, kcache: np.ndarray, vcache: np.ndarray, pos: int, n_heads: int,
              n_kv_heads: int, head_size: int) -> np.ndarray:
    """runq.c:367-391 over caches laid out [n_kv_heads][max_t][head_size]."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    kc = np.ascontiguousarray(kcache, dtype=np.float32)
    vc = np.ascontiguousarray(vcache, dtype=np.float32)
    max_t = kc.shape[1]
    out = np.empty(n_heads * head_size, dtype=np.float32)
    att = np.empty(n_heads * (pos + 1), dtype=np.float32)
    olib().orc_attention(_p(q), _p(kc), _p(vc), _p(out), pos, n_heads, n_kv_heads, head_size,
                         head_size, max_t * head_size, _p(att), pos + 1)
    return out


def kv_quant(row: np.ndarray):
    """(int8 row, scale) of one kv head (v5-cuda-fused/run.cu:204-249)."""
    row = np.ascontiguousarray(row, dtype=np.float32)
    q = np.empty(row.size, dtype=np.int8)
    s = np.empty(1, dtype=np.float32)
    olib().orc_kv_quant(_p(row), row.size, _p(q), _p(s))
    return q, np.float32(s[0])


def attention_kv8(q: np.ndarray, k8: np.ndarray, v8: np.ndarray, ks: np.ndarray, vs: np.ndarray, pos: int,
                  n_heads: int, n_kv_heads: int, head_size: int, ordered: bool = False,
                  splits: int = 0) -> np.ndarray:
    """v5-cuda-fused/run.cu:350-410 (in double, with ordered=True in the
    one-workgroup GPU kernel's float order, with splits=S in the split
    kernel's) over int8 caches laid out [n_kv_heads][max_t][head_size] with
    scales [n_kv_heads][max_t]."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k8 = np.ascontiguousarray(k8, dtype=np.int8)
    v8 = np.ascontiguousarray(v8, dtype=np.int8)
    ks = np.ascontiguousarray(ks, dtype=np.float32)
    vs = np.ascontiguousarray(vs, dtype=np.float32)
    max_t = k8.shape[1]
    out = np.empty(n_heads * head_size, dtype=np.float32)
    args = (_p(q), _p(k8), _p(v8), _p(ks), _p(vs), _p(out), pos, n_heads, n_kv_heads, head_size,
            head_size, max_t * head_size, 1, max_t)
    if splits:
        olib().orc_attention_kv8_split(*args, splits)
    else:
        (olib().orc_attention_kv8_ordered if ordered else olib().orc_attention_kv8)(*args)
    return out


def swiglu(h: np.ndarray, h2: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.float32)
    h2 = np.ascontiguousarray(h2, dtype=np.float32)
    out = np.empty_like(h)
    olib().orc_swiglu(_p(out), _p(h), _p(h2), h.size)
    return out


def expf_host(x: np.ndarray) -> np.ndarray:
    """The host C library's expf, elementwise."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    olib().orc_expf_array(_p(x), _p(y), x.size)
    return y


class Oracle:
    """CPU restatement of forward() over a checkpoint image (host memory)."""

    def __init__(self, cfg_list, weights: np.ndarray, wbits: int, group: int, max_t: int = 0, kv8: bool = False,
                 kv8_splits: int = 0, kv8_split_from: int = 0):
        """kv8: the int8 KV cache; kv8_splits > 0: its attention over more
        than kv8_split_from positions in the split kernel's order with that
        many splits (the one-workgroup order below, and everywhere with 0)."""
        self.cfg = list(cfg_list)
        self.dim, self.n_layers, self.vocab = self.cfg[0], self.cfg[2], self.cfg[5]
        self._w = weights   # keep the buffer alive
        arr = (C.c_int * 7)(*self.cfg)
        self._m = olib().orc_model_create(arr, _p(weights), weights.nbytes, wbits, group, max_t)
        if not self._m:
            raise ValueError("oracle: weights image too short for the config")
        if kv8 and olib().orc_model_set_kv8(self._m, 1) != 0:
            raise MemoryError("oracle: int8 KV cache")
        if kv8 and olib().orc_model_set_kv8_splits(self._m, kv8_splits, kv8_split_from) != 0:
            raise ValueError("oracle: splits outside 0..64")

    def forward(self, token: int, pos: int, layers: bool = False):
        xl = np.empty((self.n_layers + 1, self.dim), dtype=np.float32) if layers else None
        ptr = olib().orc_forward(self._m, token, pos, _p(xl))
        logits = np.ctypeslib.as_array(ptr, shape=(self.vocab,)).copy()
        return (xl, logits) if layers else logits

    def greedy(self, prompt, n_steps: int):
        pr = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.empty(n_steps, dtype=np.int32)
        olib().orc_greedy(self._m, _p(pr), len(pr), n_steps, _p(out))
        return [int(v) for v in out]

    def close(self):
        if self._m:
            olib().orc_model_free(self._m)
            self._m = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---------------------------------------------------------------------------
# the reference runner compiled from its own source


def ref_available() -> bool:
    return os.path.exists(REF_LIB)


_rlib = None


def rlib():
    global _rlib
    if _rlib is None:
        L = C.CDLL(REF_LIB)
        sig = {
            "ref_open": (I, [C.c_char_p]),
            "ref_open_memory": (I, [P, C.c_size_t]),
            "ref_config": (None, [P]),
            "ref_forward": (C.POINTER(C.c_float), [I, I]),
            "ref_close": (None, []),
            "ref_quantize_act": (None, [P, I, P, P, P]),
            "ref_matmul_q8": (None, [P, P, P, P, P, P, I, I]),
            "ref_rmsnorm": (None, [P, P, P, I]),
            "ref_softmax": (None, [P, I]),
            "ref_sample_argmax": (I, [P, I]),
            "ref_tok_open": (None, [C.c_char_p, I]),
            "ref_tok_encode": (I, [C.c_char_p, I, I, P]),
            "ref_tok_decode": (C.c_char_p, [I, I]),
            "ref_tok_close": (None, []),
            "ref_sampler_open": (None, [I, C.c_float, C.c_float, C.c_ulonglong]),
            "ref_sample": (I, [P]),
            "ref_sampler_state": (C.c_ulonglong, []),
            "ref_sampler_close": (None, []),
        }
        for n, (r, a) in sig.items():
            f = getattr(L, n)
            f.restype = r
            f.argtypes = a
        _rlib = L
    return _rlib


class RefRunq:
    """runq.c's Transformer on a QLL8 (version 1, group 32) file, or on a
    checkpoint image in memory (``image``: uint8 array of a whole file)."""

    def __init__(self, path: str = None, image: np.ndarray = None):
        if image is not None:
            self._image = image
            self.vocab = rlib().ref_open_memory(_p(image), image.nbytes)
            if self.vocab < 0:
                raise ValueError("not a QLL8 version-1 image")
        else:
            self.vocab = rlib().ref_open(path.encode())
        cfg = np.empty(7, dtype=np.int32)
        rlib().ref_config(_p(cfg))
        self.cfg = [int(v) for v in cfg]

    def forward(self, token: int, pos: int) -> np.ndarray:
        ptr = rlib().ref_forward(token, pos)
        return np.ctypeslib.as_array(ptr, shape=(self.vocab,)).copy()

    def greedy(self, prompt, n_steps: int):
        ids, token = [], prompt[0]
        for pos in range(n_steps):
            lg = self.forward(token, pos)
            nxt = prompt[pos + 1] if pos < len(prompt) - 1 else int(np.argmax(lg))
            ids.append(int(nxt))
            token = nxt
        return ids

    def close(self):
        rlib().ref_close()


def ref_argmax(v: np.ndarray) -> int:
    v = np.ascontiguousarray(v, dtype=np.float32).copy()
    return int(rlib().ref_sample_argmax(_p(v), v.size))


def ref_quantize_act(x: np.ndarray):
    x = np.ascontiguousarray(x, dtype=np.float32)
    n = x.size
    xq = np.empty(n, dtype=np.int8)
    xs = np.empty(n // 32, dtype=np.float32)
    xt = np.empty(n // 32, dtype=np.float32)
    rlib().ref_quantize_act(_p(x), n, _p(xq), _p(xs), _p(xt))
    return xq, xs, xt


def ref_matmul_q8(xq, xs, xt, w_u8, ws, rows: int, cols: int) -> np.ndarray:
    out = np.empty(rows, dtype=np.float32)
    xq, xs, xt = (np.ascontiguousarray(a) for a in (xq, xs, xt))
    w_u8, ws = np.ascontiguousarray(w_u8), np.ascontiguousarray(ws)
    rlib().ref_matmul_q8(_p(out), _p(xq), _p(xs), _p(xt), _p(w_u8), _p(ws), rows, cols)
    return out


def ref_rmsnorm(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).copy()
    w = np.ascontiguousarray(w, dtype=np.float32).copy()
    o = np.empty_like(x)
    rlib().ref_rmsnorm(_p(o), _p(x), _p(w), x.size)
    return o


class RefTokenizer:
    """runq.c's build_tokenizer / encode / decode."""

    def __init__(self, path: str, vocab_size: int):
        rlib().ref_tok_open(path.encode(), vocab_size)

    def encode(self, text: str, bos: bool = True, eos: bool = False):
        b = text.encode()
        out = np.empty(len(b) + 3, dtype=np.int32)
        n = rlib().ref_tok_encode(b, int(bos), int(eos), _p(out))
        return [int(v) for v in out[:n]]

    def decode(self, prev: int, token: int) -> bytes:
        return rlib().ref_tok_decode(prev, token)

    def close(self):
        rlib().ref_tok_close()


class RefSampler:
    """runq.c's build_sampler / sample."""

    def __init__(self, vocab_size: int, temperature: float, topp: float, seed: int):
        rlib().ref_sampler_open(vocab_size, temperature, topp, seed)

    def sample(self, logits: np.ndarray) -> int:
        buf = np.ascontiguousarray(logits, dtype=np.float32).copy()
        return rlib().ref_sample(_p(buf))

    @property
    def rng_state(self) -> int:
        return rlib().ref_sampler_state()

    def close(self):
        rlib().ref_sampler_close()

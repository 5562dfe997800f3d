"""ctypes binding of build/libl2q.so (include/l2q.h).

Device pointers are passed as integers (e.g. ``tensor.data_ptr()``) and
streams as integers (``torch.cuda.current_stream().cuda_stream``); nothing
here depends on torch.
"""
import ctypes as C
import os

from . import GPU_LIB

L2Q_OK = 0
L2Q_ERR_ARG = -1
L2Q_ERR_HIP = -2
L2Q_ERR_FORMAT = -3
L2Q_ERR_NOMEM = -4
L2Q_ERR_STATE = -5
L2Q_ENGINE_KV_INT8 = 1
L2Q_ENGINE_STEP_KERNEL = 2
L2Q_ENGINE_ATTN_SPLIT = 4
L2Q_KV8_SPLIT_FROM = 1024
L2Q_ATTN_SPLIT_FROM = 320
L2Q_ATTN_K_INTERLEAVED = 1
L2Q_ATTN_ONE_KERNEL = 2
L2Q_ATTN_TWO_KERNELS = 4
L2Q_ATTN_SPLIT_CONTEXT = 8
L2Q_GEMV_QKV, L2Q_GEMV_WO, L2Q_GEMV_W13, L2Q_GEMV_W2, L2Q_GEMV_CLASSIFIER = range(5)


class L2QError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"l2q error {code}: {msg}")
        self.code = code


class Config(C.Structure):
    _fields_ = [(n, C.c_int) for n in
                ("dim", "hidden_dim", "n_layers", "n_heads", "n_kv_heads", "vocab_size", "seq_len")]

    def as_list(self):
        return [getattr(self, n) for n, _ in self._fields_]


P = C.c_void_p
I = C.c_int
# name -> (restype, argtypes); the full exported surface of include/l2q.h
SIGNATURES = {
    "l2q_last_error": (C.c_char_p, []),
    "l2q_device_count": (I, []),
    "l2q_engine_create": (I, [C.POINTER(Config), P, C.c_size_t, I, I, I, C.POINTER(P)]),
    "l2q_engine_create_ex": (I, [C.POINTER(Config), P, C.c_size_t, I, I, I, I, C.POINTER(P)]),
    "l2q_engine_forward": (I, [P, I, I, P]),
    "l2q_engine_forward_argmax": (I, [P, I, I, C.POINTER(I)]),
    "l2q_engine_forward_debug": (I, [P, I, I, P, P]),
    "l2q_engine_prefill": (I, [P, P, I, I, P]),
    "l2q_engine_time_steps": (I, [P, P, I, I, C.POINTER(C.c_double)]),
    "l2q_engine_time_gemv": (I, [P, I, I, C.POINTER(C.c_double)]),
    "l2q_engine_device_bytes": (C.c_size_t, [P]),
    "l2q_engine_uses_step_kernel": (I, [P]),
    "l2q_engine_attention_splits": (I, [P]),
    "l2q_engine_destroy": (None, [P]),
    "l2q_quantize_act": (I, [P, I, I, P, P, P]),
    "l2q_gemv_q8": (I, [P, P, P, P, P, I, I, I, P, P]),
    "l2q_gemv_q4": (I, [P, P, P, P, P, I, I, I, P, P]),
    "l2q_gemm_q": (I, [I, P, P, P, P, P, I, I, I, I, P]),
    "l2q_unbias_q8": (I, [P, P, C.c_size_t, P]),
    "l2q_rmsnorm_quant": (I, [P, P, P, P, I, I, P, P, P]),
    "l2q_swiglu_quant": (I, [P, P, I, I, P, P, P, P]),
    "l2q_rope_kv_append": (I, [P, P, P, P, P, P, I, I, I, I, I, P]),
    "l2q_attention": (I, [P, P, P, P, I, I, I, I, I, P]),
    "l2q_attention_ex": (I, [P, P, P, P, I, I, I, I, I, I, P]),
    "l2q_argmax": (I, [P, I, P, P]),
    "l2q_attention_split": (I, [P, P, P, P, I, I, I, I, I, P]),
    "l2q_attention_split_noalloc": (I, [P, P, P, P, I, I, I, I, I, P]),
    "l2q_kv8_append": (I, [P, P, P, P, P, P, P, I, I, I, I, P]),
    "l2q_attention_kv8": (I, [P, P, P, P, P, P, I, I, I, I, I, P]),
    "l2q_attention_kv8_ex": (I, [P, P, P, P, P, P, I, I, I, I, I, I, P]),
    "l2q_expf": (I, [P, P, C.c_size_t, P]),
    "l2q_rope_table": (None, [P, I, I]),
}

_lib = None


def lib():
    """Load libl2q.so once (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(GPU_LIB):
            raise RuntimeError(f"{GPU_LIB} is not built; run __graft_entry__.build() or make")
        L = C.CDLL(GPU_LIB)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def last_error() -> str:
    return lib().l2q_last_error().decode(errors="replace")


def check(rc: int) -> None:
    if rc != L2Q_OK:
        raise L2QError(rc, last_error())


def call(name: str, *args) -> None:
    """Call an int-returning entry point and raise on a failure status."""
    check(getattr(lib(), name)(*args))

"""Engine wrapper: the decode step of a QLL8/QLL4 checkpoint on one GPU.

Mirrors the reference seam ``forward(transformer, token, pos) -> logits``
(runq.c:320) and the greedy loop of runq.c:681-718, through the C ABI.
"""
import ctypes as C

import numpy as np

from . import abi
from .host import Checkpoint


class Engine:
    def __init__(self, ckpt: Checkpoint, max_steps: int = 0, kv8: bool = False, step_kernel: bool = False,
                 attn_split: bool = False):
        """kv8: int8 KV cache (L2Q_ENGINE_KV_INT8, the reference's INT8_KV build);
        step_kernel: run each step as one persistent kernel where the shape
        allows it (L2Q_ENGINE_STEP_KERNEL; same bits as the per-op graph);
        attn_split: split-context decode attention, equal to the reference
        up to rounding (L2Q_ENGINE_ATTN_SPLIT)."""
        if ckpt.header.shared_weights:
            raise ValueError("shared weights not supported")   # runq.c:247-251
        self.cfg = ckpt.cfg
        self.vocab = self.cfg.vocab_size
        w = ckpt.weights
        h = C.c_void_p()
        flags = (abi.L2Q_ENGINE_KV_INT8 if kv8 else 0) | (abi.L2Q_ENGINE_STEP_KERNEL if step_kernel else 0) | \
            (abi.L2Q_ENGINE_ATTN_SPLIT if attn_split else 0)
        abi.call("l2q_engine_create_ex", C.byref(self.cfg), w.ctypes.data, w.nbytes, ckpt.wbits, ckpt.group,
                 max_steps, flags, C.byref(h))
        self._h = h
        self.max_steps = max_steps if 0 < max_steps <= self.cfg.seq_len else self.cfg.seq_len
        self._logits = np.empty(self.vocab, dtype=np.float32)

    def forward(self, token: int, pos: int) -> np.ndarray:
        """Logits after one step (a copy owned by the caller)."""
        abi.call("l2q_engine_forward", self._h, token, pos, self._logits.ctypes.data)
        return self._logits.copy()

    def prefill(self, tokens, pos0: int, logits: bool = True):
        """Positions pos0.. take `tokens` in one batched pass; the logits of
        the last position (or None)."""
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        abi.call("l2q_engine_prefill", self._h, t.ctypes.data, t.size, pos0,
                 self._logits.ctypes.data if logits else None)
        return self._logits.copy() if logits else None

    def step(self, token: int, pos: int) -> None:
        """One step without fetching logits (prompt forcing)."""
        abi.call("l2q_engine_forward", self._h, token, pos, None)

    def forward_argmax(self, token: int, pos: int) -> int:
        out = C.c_int()
        abi.call("l2q_engine_forward_argmax", self._h, token, pos, C.byref(out))
        return out.value

    def forward_debug(self, token: int, pos: int):
        """(x after embedding and after every layer [L+1, dim], logits)."""
        xl = np.empty((self.cfg.n_layers + 1, self.cfg.dim), dtype=np.float32)
        lg = np.empty(self.vocab, dtype=np.float32)
        abi.call("l2q_engine_forward_debug", self._h, token, pos, xl.ctypes.data, lg.ctypes.data)
        return xl, lg

    def time_steps(self, tokens, pos0: int) -> float:
        """Device milliseconds for len(tokens) graph replays (no logits copy)."""
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        ms = C.c_double()
        abi.call("l2q_engine_time_steps", self._h, t.ctypes.data, pos0, len(t), C.byref(ms))
        return ms.value

    def time_gemv(self, kind: int, n_launches: int) -> float:
        """Device milliseconds for n_launches of the step's GEMV kernel of
        `kind` (abi.L2Q_GEMV_*) with the decode's arguments, rotating over
        the layers' weights; the decode state is left unchanged."""
        ms = C.c_double()
        abi.call("l2q_engine_time_gemv", self._h, kind, n_launches, C.byref(ms))
        return ms.value

    def greedy(self, prompt, n_steps: int, device_argmax: bool = True):
        """Force `prompt`, then pick argmax until n_steps positions have run.
        Returns the id chosen after every position (no BOS stop)."""
        ids = []
        token = prompt[0]
        for pos in range(n_steps):
            if pos < len(prompt) - 1:
                self.step(token, pos)
                nxt = prompt[pos + 1]
            elif device_argmax:
                nxt = self.forward_argmax(token, pos)
            else:
                nxt = int(np.argmax(self.forward(token, pos)))
            ids.append(int(nxt))
            token = nxt
        return ids

    @property
    def attention_splits(self) -> int:
        """Context splits of the decode attention (0: the exact order)."""
        return abi.lib().l2q_engine_attention_splits(self._h)

    @property
    def step_kernel(self) -> bool:
        """Whether each step runs as the one persistent kernel."""
        return bool(abi.lib().l2q_engine_uses_step_kernel(self._h))

    @property
    def device_bytes(self) -> int:
        return abi.lib().l2q_engine_device_bytes(self._h)

    def close(self):
        if getattr(self, "_h", None) and self._h.value:
            abi.lib().l2q_engine_destroy(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

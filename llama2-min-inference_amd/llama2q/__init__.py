"""llama2q - Python side of the MI355X batch-1 quantized Llama-2 decode path.

The compute lives in native code built by `make` in the package directory:

* ``build/libl2q.so`` - hand-written HIP kernels for gfx950, the op-level C
  ABI and the decode engine (declared in ``include/l2q.h``);
* ``build/libl2q_host.so`` - checkpoint format, deterministic random-init
  checkpoint writer, tokenizer and sampler (plain C);
* ``build/llama2q_run`` - the drop-in command-line runner.

This package only binds those libraries with ctypes (``abi``, ``host``) and
wraps them in small classes (``model``).  There is no Python or CPU
fallback for any GPU op: if ``libl2q.so`` is missing or no GPU is visible,
the GPU entry points raise.
"""
import os

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REPO_DIR = os.path.dirname(PKG_DIR)
BUILD_DIR = os.path.join(PKG_DIR, "build")
INCLUDE_DIR = os.path.join(REPO_DIR, "include")

GPU_LIB = os.path.join(BUILD_DIR, "libl2q.so")
HOST_LIB = os.path.join(BUILD_DIR, "libl2q_host.so")
RUNNER = os.path.join(BUILD_DIR, "llama2q_run")


def build(jobs: int = 8) -> None:
    """Compile every native target (hipcc for gfx950, gcc for the host)."""
    import subprocess

    subprocess.run(["make", "-C", PKG_DIR, f"-j{jobs}"], check=True)

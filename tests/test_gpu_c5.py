"""BASELINE config 5 at full depth: the workload bench.py times.

The Llama-2-7B-shaped INT4 group-64 model (32 layers, a 3.7 GB weight
arena) is built from the same seed as bench.py.  Its 128 prompt ids are
prefilled (positions 0..126, as the runner and the bench do), and then 256
greedy steps run through the captured step graph with the argmax on the
device (positions 127..382, the decode loop of runq.c:681-718).

The expected values are tests/golden/c5_7b_int4_g64.json, written by
tests/golden/make_c5.py from the CPU oracle (oracle/oracle.c, the
restatement of runq.c:320-421 with the tools/quantize_int4.py dequant):
  * the 256 greedy ids must be identical;
  * at positions 127, 300 and 382 the step runs as the engine's eager
    diagnostic form (the same kernels, launched one at a time) and the
    residual stream after the embedding and after each of the 32 layers,
    and the logits, must be bit-identical (sha256 of the fp32 bytes).
The checkpoint generator is pinned by the sha256 of the image's first and
last 64 MiB.  Both step forms run the case: the default graph of one kernel
per op, and the opt-in single persistent kernel (L2Q_ENGINE_STEP_KERNEL),
whose eager diagnostic form writes the per-layer residual stream from inside
the kernel.
"""
import hashlib
import json
import os
import sys

import numpy as np
import pytest

from conftest import GOLDEN
from llama2q.model import Engine
import oracle_py as O

sys.path.insert(0, GOLDEN)
import make_c5  # noqa: E402

pytestmark = pytest.mark.gpu


def sha(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


@pytest.fixture(scope="module")
def c5():
    with open(os.path.join(GOLDEN, "c5_7b_int4_g64.json")) as f:
        gold = json.load(f)
    ck = make_c5.c5_checkpoint()
    assert make_c5.image_pins(ck.weights) == gold["image"], "the synthetic checkpoint generator changed"
    assert make_c5.c5_prompt() == gold["prompt"]
    return ck, gold


@pytest.mark.parametrize("step_kernel", [False, True], ids=["graph", "step_kernel"])
def test_c5_full_depth_greedy_256_and_layers(gpu_lib, c5, step_kernel):
    ck, gold = c5
    prompt = gold["prompt"]
    n_pos = gold["n_positions"]
    eng = Engine(ck, max_steps=n_pos, step_kernel=step_kernel)
    assert eng.step_kernel == step_kernel, "the MI355X (256 CUs) runs this shape as one kernel when asked"
    eng.prefill(prompt[:-1], 0, logits=False)
    token, ids = prompt[-1], []
    for pos in range(len(prompt) - 1, n_pos):
        rec = gold["layers"].get(str(pos))
        if rec is None:
            nxt = eng.forward_argmax(token, pos)
        else:
            xl, lg = eng.forward_debug(token, pos)
            got = [sha(row) for row in xl]
            bad = [i for i, (g, w) in enumerate(zip(got, rec["x_sha256"])) if g != w]
            assert not bad, (f"pos {pos}: residual stream differs from the oracle first after "
                             f"{'the embedding' if bad[0] == 0 else f'layer {bad[0] - 1}'} "
                             f"(got {xl[bad[0], :4].tolist()}, want {rec['x_first4'][bad[0]]})")
            assert sha(lg) == rec["logits_sha256"], f"pos {pos}: logits differ"
            nxt = O.argmax(lg)
        ids.append(int(nxt))
        token = nxt
    eng.close()
    want = gold["ids"][len(prompt) - 1:]
    assert len(ids) == len(want) == 256
    first = next((i for i, (a, b) in enumerate(zip(ids, want)) if a != b), None)
    assert first is None, f"greedy id {first} (position {first + len(prompt) - 1}) differs: {ids[first]} vs {want[first]}"

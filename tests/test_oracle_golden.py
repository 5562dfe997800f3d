"""The oracle against the golden fixtures written from the compiled
reference runq.c by tests/golden/make_golden.py (runs without the
reference checkout).  Bit-exact throughout."""
import hashlib
import json
import os

import numpy as np
import pytest

from conftest import GOLDEN
from llama2q import host
import oracle_py as O


def load(name):
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


def test_ref_ops_vectors():
    g = np.load(os.path.join(GOLDEN, "ref_ops.npz"))
    xq, xs, xt = O.quantize_act(g["qa_x"], 32)
    np.testing.assert_array_equal(xq, g["qa_xq"])
    np.testing.assert_array_equal(xs, g["qa_xs"])
    np.testing.assert_array_equal(xt, g["qa_xt"])
    rows, cols = g["mm_wq"].shape
    out, _ = O.matmul(8, g["qa_xq"], g["qa_xs"], g["qa_xt"], g["mm_wq"], g["mm_ws"], rows, cols, 32)
    np.testing.assert_array_equal(out, g["mm_out"])
    np.testing.assert_array_equal(O.rmsnorm(g["rn_x"], g["rn_w"]), g["rn_out"])


def test_ref_ops_weights_regenerate():
    """The fixture's quantized weights are what the build's writer makes."""
    g = np.load(os.path.join(GOLDEN, "ref_ops.npz"))
    rows, cols = g["mm_wq"].shape
    w = host.gauss(rows * cols, 5, 2, 0.02).reshape(rows, cols)
    q, s = host.quantize_q8(w, 32)
    np.testing.assert_array_equal(q, g["mm_wq"])
    np.testing.assert_array_equal(s, g["mm_ws"])


@pytest.fixture(scope="module")
def c1():
    gold = load("c1_q8_greedy.json")
    cfg = host.config_15m()
    assert gold["config"] == cfg.as_list()
    ck = host.synth_checkpoint(cfg, 8, 32, seed=gold["seed"], sigma=gold["sigma"])
    return gold, ck


def test_c1_checkpoint_bytes(c1):
    gold, ck = c1
    assert hashlib.sha256(ck.data.tobytes()).hexdigest() == gold["checkpoint_sha256"]
    assert gold["prompt"] == [int(v) for v in host.uniform_ints(16, gold["seed"], 100, 3, 32000)]


def test_c1_greedy_ids_and_logits(c1):
    gold, ck = c1
    orc = O.Oracle(ck.cfg.as_list(), ck.weights, 8, 32, max_t=256)
    full = np.load(os.path.join(GOLDEN, "c1_q8_logits.npz"))
    token = gold["prompt"][0]
    ids = []
    for pos in range(256):
        lg = orc.forward(token, pos)
        if f"step{pos}" in full:
            np.testing.assert_array_equal(lg, full[f"step{pos}"])
        if str(pos) in gold["top8"]:
            for i, v in gold["top8"][str(pos)]:
                assert lg[i] == np.float32(v)
        nxt = gold["prompt"][pos + 1] if pos < 15 else int(np.argmax(lg))
        ids.append(nxt)
        token = nxt
    assert ids == gold["ids"]


def test_c1_int4_lifted_greedy():
    gold = load("c1_q4_lifted.json")
    cfg = host.config_15m()
    ck = host.synth_checkpoint(cfg, 4, 32, seed=gold["seed"], q4_divisor=gold["divisor"])
    assert hashlib.sha256(ck.data.tobytes()).hexdigest() == gold["checkpoint_sha256"]
    orc = O.Oracle(cfg.as_list(), ck.weights, 4, 32, max_t=256)
    assert orc.greedy(gold["prompt"], 256) == gold["ids"]

"""The oracle against the reference itself: v1-int8-vnni/runq.c compiled
unmodified from the reference checkout (oracle/_ref, built by
oracle/Makefile).  Every comparison is bit-exact.  Skipped where the
reference build is absent (the golden fixtures of test_oracle_golden.py
carry the same checks there).
"""
import numpy as np
import pytest

from llama2q import host
import oracle_py as O

pytestmark = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (no reference checkout)")


@pytest.fixture(scope="module")
def c1_q8():
    return host.synth_checkpoint(host.config_15m(), 8, 32, seed=1234)


def test_quantize_act_bit_exact():
    for seed in range(5):
        x = host.gauss(768, seed, 1, 1.0 + seed)
        x[32:64] = 0.0
        x[64] = 0.5
        got = O.quantize_act(x, 32)
        ref = O.ref_quantize_act(x)
        for g, r in zip(got, ref):
            np.testing.assert_array_equal(g, r)


def test_argmax_equals_reference_scan():
    """orc_argmax against runq.c's sample_argmax, including the cases where
    the scan from v[0] differs from numpy's argmax (NaNs skipped, a NaN at
    index 0, all -inf, ties)."""
    rng = np.random.default_rng(4)
    cases = []
    for n in (1, 5, 32000):
        v = rng.standard_normal(n).astype(np.float32)
        cases.append(v)
        w = v.copy(); w[rng.integers(0, n, size=min(n, 4))] = np.float32(9.0); cases.append(w)
        w = v.copy(); w[rng.integers(0, n, size=min(n, 4))] = np.nan; cases.append(w)
        w = v.copy(); w[0] = np.nan; cases.append(w)
        cases.append(np.full(n, -np.inf, np.float32))
        cases.append(np.full(n, np.nan, np.float32))
    for v in cases:
        assert O.argmax(v) == O.ref_argmax(v), v[:6]


@pytest.mark.parametrize("rows,cols", [(64, 288), (96, 768), (17, 4096)])
def test_matmul_q8_bit_exact(rows, cols):
    w = host.gauss(rows * cols, rows, 2, 0.02).reshape(rows, cols)
    wq, ws = host.quantize_q8(w, 32)
    x = host.gauss(cols, rows, 3, 1.0)
    xq, xs, xt = O.quantize_act(x, 32)
    out, dots = O.matmul(8, xq, xs, xt, wq, ws, rows, cols, 32)
    np.testing.assert_array_equal(out, O.ref_matmul_q8(xq, xs, xt, wq, ws, rows, cols))
    # signed int32 group dots: an independent integer product
    wsgn = wq.astype(np.int64) - 128
    exp = (wsgn.reshape(rows, cols // 32, 32) * xq.astype(np.int64).reshape(1, cols // 32, 32)).sum(-1)
    np.testing.assert_array_equal(dots, exp)


@pytest.mark.parametrize("n", [288, 4096, 4104, 4100])
def test_rmsnorm_bit_exact(n):
    x = host.gauss(n, n, 4, 1.0)
    w = (1.0 + host.gauss(n, n, 5, 0.1)).astype(np.float32)
    np.testing.assert_array_equal(O.rmsnorm(x, w), O.ref_rmsnorm(x, w))


def test_forward_c1_bit_exact(c1_q8, tmp_path):
    path = str(tmp_path / "c1.bin")
    c1_q8.save(path)
    ref = O.RefRunq(path)
    orc = O.Oracle(c1_q8.cfg.as_list(), c1_q8.weights, 8, 32)
    prompt = [int(v) for v in host.uniform_ints(16, 1234, 100, 3, 32000)]
    token = prompt[0]
    for pos in range(48):
        a = ref.forward(token, pos)
        b = orc.forward(token, pos)
        np.testing.assert_array_equal(a, b)
        token = prompt[pos + 1] if pos < 15 else int(np.argmax(a))
    ref.close()


def test_forward_from_memory_equals_file(c1_q8, tmp_path):
    path = str(tmp_path / "c1.bin")
    c1_q8.save(path)
    a = O.RefRunq(path)
    la = [a.forward(7, p) for p in range(3)]
    a.close()
    b = O.RefRunq(image=c1_q8.data)
    lb = [b.forward(7, p) for p in range(3)]
    b.close()
    for x, y in zip(la, lb):
        np.testing.assert_array_equal(x, y)


def test_int4_oracle_equals_runq_on_lifted_model(tmp_path):
    """An INT4 model run through the INT4 oracle equals runq.c on the same
    model with every int4 value stored as int8 (same scales)."""
    import sys
    sys.path.insert(0, str(__import__("pathlib").Path(__file__).parent / "golden"))
    from make_golden import lift_q4_to_q8
    cfg = host.config_15m()
    ck4 = host.synth_checkpoint(cfg, 4, 32, seed=5, q4_divisor=8.0)
    lifted = lift_q4_to_q8(ck4)
    ref = O.RefRunq(image=lifted)
    orc = O.Oracle(cfg.as_list(), ck4.weights, 4, 32)
    token = 300
    for pos in range(24):
        a = ref.forward(token, pos)
        b = orc.forward(token, pos)
        np.testing.assert_array_equal(a, b)
        token = int(np.argmax(a))
    ref.close()


def tokenizer_file(tmp_path):
    pieces, scores = host.synth_tokenizer_pieces(32000)
    path = str(tmp_path / "tok.bin")
    host.write_tokenizer(path, pieces, scores)
    return path


@pytest.mark.parametrize("text", ["", "Once upon a time", "hello world", "[INST] hi [/INST]",
                                  "naïve café ☃", "a" * 40, " leading space", "x\ny\tz"])
def test_tokenizer_matches_reference(tmp_path, text):
    path = tokenizer_file(tmp_path)
    ours = host.Tokenizer(path, 32000)
    ref = O.RefTokenizer(path, 32000)
    for bos, eos in [(1, 0), (0, 0), (1, 1)]:
        assert ours.encode(text, bool(bos), bool(eos)) == ref.encode(text, bool(bos), bool(eos))
    ids = ours.encode(text)
    for prev, tok in zip([1] + ids, ids + [300]):
        assert ours.decode(prev, tok) == ref.decode(prev, tok)
    ours.close()
    ref.close()


@pytest.mark.parametrize("temperature,topp", [(0.0, 0.9), (1.0, 0.9), (0.7, 0.95), (1.3, 1.0), (0.9, 0.0)])
def test_sampler_matches_reference(temperature, topp):
    ours = host.Sampler(32000, temperature, topp, 1234)
    ref = O.RefSampler(32000, temperature, topp, 1234)
    for i in range(20):
        logits = host.gauss(32000, 77, i, 2.0)
        assert ours.sample(logits) == ref.sample(logits)
        assert ours.rng_state == ref.rng_state
    ref.close()

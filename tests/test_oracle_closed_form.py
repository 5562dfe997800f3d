"""Pins of the oracle (and of the offline quantizers) that do not depend on
the reference build: closed forms, brute force on small inputs, special
cases and invariants.  These are what pin group size 64 (the reference is
fixed at 32) and the INT4 path (the reference has no CPU INT4 runner).

A plausible mistake - a swapped nibble order, a dropped bias term, a wrong
rounding mode, a transposed scale - fails at least one of these.
"""
import numpy as np
import pytest

from llama2q import host
import oracle_py as O


def unpack_q4(packed: np.ndarray) -> np.ndarray:
    """Two's-complement nibbles, low nibble = even column (numpy bit ops)."""
    lo = (packed & 0x0F).astype(np.int16)
    hi = (packed >> 4).astype(np.int16)
    lo = np.where(lo > 7, lo - 16, lo)
    hi = np.where(hi > 7, hi - 16, hi)
    out = np.empty(packed.shape[:-1] + (packed.shape[-1] * 2,), dtype=np.int16)
    out[..., 0::2] = lo
    out[..., 1::2] = hi
    return out


# ---------------------------------------------------------------- quantizers

@pytest.mark.parametrize("group", [32, 64])
def test_activation_quantizer_properties(group):
    x = host.gauss(64 * group, 3, 1, 2.0)
    x[:group] = 0.0
    xq, xs, xt = O.quantize_act(x, group)
    xb = x.reshape(-1, group)
    amax = np.abs(xb).max(1)
    np.testing.assert_array_equal(xs[1:], (amax[1:] / np.float32(127.0)).astype(np.float32))
    assert xs[0] == np.float32(1e-8) and not xq[:group].any()          # zero group
    qb = xq.reshape(-1, group).astype(np.int64)
    # the largest element of each group maps to +-127 exactly
    idx = np.abs(xb).argmax(1)
    assert (np.abs(qb[np.arange(len(idx)), idx])[1:] == 127).all()
    # q = round-half-even(x / s) computed in float32
    ratio = (xb / xs[:, None]).astype(np.float32)
    np.testing.assert_array_equal(qb, np.clip(np.rint(ratio), -127, 127))
    # the bias term is s * 128 * sum(q) in float32
    np.testing.assert_array_equal(xt, (xs * np.float32(128.0) * qb.sum(1).astype(np.float32)).astype(np.float32))


def test_activation_quantizer_ties_round_to_even():
    x = np.zeros(32, dtype=np.float32)
    x[0] = 127.0                       # scale exactly 1.0
    x[1:6] = [0.5, 1.5, 2.5, -0.5, -2.5]
    xq, xs, _ = O.quantize_act(x, 32)
    assert xs[0] == 1.0
    assert list(xq[1:6]) == [0, 2, 2, 0, -2]


@pytest.mark.parametrize("divisor", [7.0, 8.0])
@pytest.mark.parametrize("group", [32, 64])
def test_int4_quantizer_closed_form(divisor, group):
    rows, cols = 12, 256
    w = host.gauss(rows * cols, 9, 1, 0.02).reshape(rows, cols)
    w[0, :group] = 0.0
    q, s = host.quantize_q4(w, group, divisor)
    wb = w.reshape(rows, cols // group, group)
    amax = np.abs(wb).max(-1)
    exp_s = (amax / np.float32(divisor)).astype(np.float32)
    exp_s[exp_s == 0] = np.float32(1e-8)
    np.testing.assert_array_equal(s, exp_s)
    exp_q = np.clip(np.rint((wb / exp_s[..., None]).astype(np.float32)), -8, 7).reshape(rows, cols)
    np.testing.assert_array_equal(unpack_q4(q), exp_q)
    assert not unpack_q4(q)[0, :group].any()
    if divisor == 7.0:
        assert unpack_q4(q).min() >= -7          # /7: -8 never occurs
    else:                                        # /8: +amax is clipped to 7, -amax is -8
        i = np.argmax(w[1])
        assert unpack_q4(q)[1, i] == (7 if w[1, i] > 0 else -8)


def test_int4_nibble_order():
    w = np.zeros((1, 64), dtype=np.float32)
    w[0, 0], w[0, 1] = 0.7, -0.8                 # amax 0.8 -> scale 0.1 (divisor 8)
    q, s = host.quantize_q4(w, 32, 8.0)
    assert q[0, 0] == (7 | (0x8 << 4))           # column 0 in the low nibble, column 1 (-8) in the high


def test_int8_quantizer_closed_form():
    rows, cols = 8, 128
    w = host.gauss(rows * cols, 4, 1, 0.02).reshape(rows, cols)
    q, s = host.quantize_q8(w, 32)
    wb = w.reshape(rows, -1, 32)
    exp_s = (np.abs(wb).max(-1) / np.float32(127.0)).astype(np.float32)
    np.testing.assert_array_equal(s, exp_s)
    exp_q = np.clip(np.rint((wb / exp_s[..., None]).astype(np.float32)), -127, 127).reshape(rows, cols) + 128
    np.testing.assert_array_equal(q, exp_q.astype(np.uint8))


# ---------------------------------------------------------------- GEMV

@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("group", [32, 64])
def test_gemv_dots_brute_force_and_float_closed_form(bits, group):
    rows, cols = 40, 640
    w = host.gauss(rows * cols, 6, 1, 0.02).reshape(rows, cols)
    x = host.gauss(cols, 6, 2, 1.0)
    xq, xs, xt = O.quantize_act(x, group)
    if bits == 8:
        q, s = host.quantize_q8(w, group)
        wi = q.astype(np.int64) - 128
    else:
        q, s = host.quantize_q4(w, group, 7.0)
        wi = unpack_q4(q).astype(np.int64)
    out, dots = O.matmul(bits, xq, xs, xt, q, s, rows, cols, group)
    nb = cols // group
    exp_dots = (wi.reshape(rows, nb, group) * xq.astype(np.int64).reshape(1, nb, group)).sum(-1)
    np.testing.assert_array_equal(dots, exp_dots)
    # float64 closed form sum_b ws * xs * dot: the reference's biased formula
    # is the same number up to float32 rounding
    exact = (s.astype(np.float64) * xs.astype(np.float64)[None, :] * exp_dots).sum(1)
    scale = (np.abs(s.astype(np.float64) * xs[None, :] * exp_dots)).sum(1)
    assert (np.abs(out - exact) <= 1e-5 * scale + 1e-12).all()


# ---------------------------------------------------------------- norm / softmax / rope / attention

@pytest.mark.parametrize("n", [288, 4096])
def test_rmsnorm_closed_form(n):
    x = host.gauss(n, 1, 1, 3.0)
    w = (1.0 + host.gauss(n, 1, 2, 0.1)).astype(np.float32)
    o = O.rmsnorm(x, w)
    xd = x.astype(np.float64)
    exact = w * xd / np.sqrt((xd * xd).mean() + 1e-5)
    np.testing.assert_allclose(o, exact, rtol=2e-6, atol=1e-7)


def test_softmax_closed_form():
    x = host.gauss(1000, 2, 1, 4.0)
    p = O.softmax(x)
    e = np.exp(x.astype(np.float64) - x.max())
    np.testing.assert_allclose(p, e / e.sum(), rtol=1e-5, atol=1e-9)
    assert abs(p.astype(np.float64).sum() - 1.0) < 1e-5
    assert np.argmax(p) == np.argmax(x)


def test_rope_properties():
    hs, dim = 128, 4096
    q = host.gauss(dim, 3, 1, 1.0)
    k = host.gauss(dim, 3, 2, 1.0)
    q0, k0 = O.rope(q, k, 0, hs)
    np.testing.assert_array_equal(q0, q)          # angle 0 is the identity
    np.testing.assert_array_equal(k0, k)
    pos = 1000
    qr, _ = O.rope(q, k, pos, hs)
    i = np.arange(0, dim, 2)
    freq = 1.0 / np.power(10000.0, (i % hs) / hs)
    ang = pos * freq
    c, s_ = np.cos(ang), np.sin(ang)
    a, b = q[0::2].astype(np.float64), q[1::2].astype(np.float64)
    np.testing.assert_allclose(qr[0::2], a * c - b * s_, atol=2e-4)
    np.testing.assert_allclose(qr[1::2], a * s_ + b * c, atol=2e-4)
    np.testing.assert_allclose(np.hypot(qr[0::2], qr[1::2]), np.hypot(a, b), rtol=1e-5)


def test_rope_table_matches_rotation_angles():
    t = O.rope_table(8, 48).reshape(8, 24, 2)
    np.testing.assert_array_equal(t[0, :, 0], 1.0)
    np.testing.assert_array_equal(t[0, :, 1], 0.0)
    np.testing.assert_allclose(t[..., 0] ** 2 + t[..., 1] ** 2, 1.0, rtol=1e-6)


@pytest.mark.parametrize("n_heads,n_kv,hs,pos", [(6, 6, 48, 0), (6, 6, 48, 37), (8, 2, 64, 100)])
def test_attention_closed_form(n_heads, n_kv, hs, pos):
    max_t = pos + 3
    kc = host.gauss(n_kv * max_t * hs, 4, 1, 1.0).reshape(n_kv, max_t, hs)
    vc = host.gauss(n_kv * max_t * hs, 4, 2, 1.0).reshape(n_kv, max_t, hs)
    q = host.gauss(n_heads * hs, 4, 3, 1.0)
    out = O.attention(q, kc, vc, pos, n_heads, n_kv, hs)
    exp = np.empty_like(out, dtype=np.float64)
    for h in range(n_heads):
        g = h // (n_heads // n_kv)
        sc = kc[g, :pos + 1].astype(np.float64) @ q[h * hs:(h + 1) * hs] / np.sqrt(hs)
        p = np.exp(sc - sc.max())
        p /= p.sum()
        exp[h * hs:(h + 1) * hs] = p @ vc[g, :pos + 1]
    np.testing.assert_allclose(out, exp, rtol=1e-5, atol=1e-6)
    if pos == 0:                                  # one position: the output is v_0 exactly
        for h in range(n_heads):
            g = h // (n_heads // n_kv)
            np.testing.assert_array_equal(out[h * hs:(h + 1) * hs], vc[g, 0])


def test_swiglu_closed_form():
    h = host.gauss(768, 5, 1, 3.0)
    h2 = host.gauss(768, 5, 2, 1.0)
    g = O.swiglu(h, h2)
    hd = h.astype(np.float64)
    np.testing.assert_allclose(g, hd / (1 + np.exp(-hd)) * h2, rtol=1e-6, atol=1e-7)


def test_expf_restatement_equals_host_expf_everywhere():
    """The exp used on the GPU (csrc/exp_runq.h, built for the host here)
    equals the host C library's expf on all 2^32 inputs."""
    lib = host.lib()
    import ctypes as C
    f = lib.l2q_exp_runq_mismatches
    f.restype = C.c_longlong
    f.argtypes = [C.c_uint64, C.c_uint64]
    assert f(0, 1 << 32) == 0


# ---------------------------------------------------------------- forward

def test_forward_first_position_closed_form():
    """At position 0 attention returns v_0, so a 1-layer model's logits can be
    rebuilt from the oracle's own ops in numpy order; the oracle's forward
    must agree to float rounding, and the KV-independent parts exactly."""
    cfg = host.make_config(64, 128, 1, 2, 2, 256, 8)
    ck = host.synth_checkpoint(cfg, 8, 32, seed=3)
    orc = O.Oracle(cfg.as_list(), ck.weights, 8, 32)
    lay = ck.layout()
    W = ck.weights
    d, hdim, V = 64, 128, 256
    f32 = lambda off, n: W[off:off + 4 * n].view(np.float32)

    def qmat(name, rows, cols):
        q = W[getattr(lay, name):getattr(lay, name) + rows * cols].reshape(rows, cols)
        s = f32(getattr(lay, name + "_s"), rows * cols // 32).reshape(rows, cols // 32)
        return q, s

    def mm(name, rows, cols, xin):
        q, s = qmat(name, rows, cols)
        xq, xs, xt = O.quantize_act(xin, 32)
        return O.matmul(8, xq, xs, xt, q, s, rows, cols, 32, want_dots=False)[0]

    tok = 17
    x = f32(lay.emb, V * d).reshape(V, d)[tok].copy()
    xb = O.rmsnorm(x, f32(lay.rms_att, d))
    v = mm("wv", d, d, xb)
    att = v                                            # pos 0: softmax weight 1 on v_0
    x = (x + mm("wo", d, d, att)).astype(np.float32)
    xb = O.rmsnorm(x, f32(lay.rms_ffn, d))
    g = O.swiglu(mm("w1", hdim, d, xb), mm("w3", hdim, d, xb))
    x = (x + mm("w2", d, hdim, g)).astype(np.float32)
    logits = mm("wcls", V, d, O.rmsnorm(x, f32(lay.rms_final, d)))
    np.testing.assert_array_equal(orc.forward(tok, 0), logits)

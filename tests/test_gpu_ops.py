"""Op-level parity on the GPU: every HIP op through the C ABI against the
CPU oracle on the same seeded inputs.

The oracle reproduces the compiled reference runq.c bit for bit, and every
GPU op evaluates the reference's arithmetic in the reference's order, so
the bar is bit-exact for all of them: int32 group dots, Q8 activations,
GEMV fp32 outputs, RMSNorm, SwiGLU, RoPE/KV append and attention.  The
split-context attention (a throughput variant with a different summation
order) is held to 1e-5 relative with an absolute floor of the output RMS.
"""
import numpy as np
import pytest

from conftest import assert_close, rel_err
from llama2q import abi, host
import oracle_py as O

pytestmark = pytest.mark.gpu

GEMV_SHAPES = [(4096, 4096), (11008, 4096), (4096, 11008), (32000, 4096)]   # c2 / c3
SMALL_SHAPES = [(288, 288), (768, 288), (288, 768), (130, 4224), (3, 64), (1, 11008)]


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def stream(torch):
    return torch.cuda.current_stream().cuda_stream


def make_weights(rows, cols, bits, group, seed, divisor=7.0):
    w = host.gauss(rows * cols, seed, 7, 0.02).reshape(rows, cols)
    if bits == 8:
        q, s = host.quantize_q8(w, group)
    else:
        q, s = host.quantize_q4(w, group, divisor)
    return q, s


def run_gemv(torch, bits, group, q, s, xq, xs, rows, cols):
    wq = q.view(np.int8) ^ np.int8(-128) if bits == 8 else q      # un-biased signed int8
    d_w, d_s = dev(torch, wq), dev(torch, s)
    d_xq, d_xs = dev(torch, xq), dev(torch, xs)
    out = torch.empty(rows, dtype=torch.float32, device="cuda")
    dots = torch.empty(rows * (cols // group), dtype=torch.int32, device="cuda")
    name = "l2q_gemv_q8" if bits == 8 else "l2q_gemv_q4"
    abi.call(name, out.data_ptr(), d_xq.data_ptr(), d_xs.data_ptr(), d_w.data_ptr(), d_s.data_ptr(),
             rows, cols, group, dots.data_ptr(), stream(torch))
    torch.cuda.synchronize()
    return out.cpu().numpy(), dots.cpu().numpy().reshape(rows, cols // group)


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("group", [32, 64])
@pytest.mark.parametrize("shape", GEMV_SHAPES + SMALL_SHAPES)
def test_gemv_matches_oracle(gpu_lib, torch_cuda, bits, group, shape):
    rows, cols = shape
    if cols % group:
        pytest.skip("group does not divide cols")
    print(f"gemv bits={bits} group={group} shape={shape}", flush=True)
    seed = 1000 * bits + group + rows
    q, s = make_weights(rows, cols, bits, group, seed)
    x = host.gauss(cols, seed, 9, 1.0)
    xq, xs, xt = O.quantize_act(x, group)
    ref, ref_dots = O.matmul(bits, xq, xs, xt, q, s, rows, cols, group)
    out, dots = run_gemv(torch_cuda, bits, group, q, s, xq, xs, rows, cols)
    np.testing.assert_array_equal(dots, ref_dots)
    np.testing.assert_array_equal(out, ref)


def test_gemv_int4_extremes(gpu_lib, torch_cuda):
    """Nibbles 0x8 (-8) and 0x7 (+7) against activations +-127."""
    rows, cols, group = 64, 4096, 64
    rng = np.random.default_rng(5)
    q = rng.choice(np.array([0x88, 0x77, 0x87, 0x78, 0x00, 0xF1], dtype=np.uint8), size=(rows, cols // 2))
    s = np.full((rows, cols // group), 0.01, dtype=np.float32)
    xq = rng.choice(np.array([127, -127, 0, 1, -1], dtype=np.int8), size=cols)
    xs = np.full(cols // group, 0.02, dtype=np.float32)
    xt = (xs * 128.0 * xq.reshape(-1, group).sum(1).astype(np.float32)).astype(np.float32)
    ref, ref_dots = O.matmul(4, xq, xs, xt, q, s, rows, cols, group)
    out, dots = run_gemv(torch_cuda, 4, group, q, s, xq, xs, rows, cols)
    np.testing.assert_array_equal(dots, ref_dots)
    np.testing.assert_array_equal(out, ref)


@pytest.mark.parametrize("group", [32, 64])
@pytest.mark.parametrize("n", [288, 768, 4096, 11008])
def test_quantize_act_bit_exact(gpu_lib, torch_cuda, group, n):
    if n % group:
        pytest.skip("group does not divide n")
    x = host.gauss(n, 77, n, 1.0)
    x[:group] = 0.0                      # an all-zero group -> scale 1e-8
    x[group] = 0.5                       # exact ties for the rounding checks
    xq_ref, xs_ref, _ = O.quantize_act(x, group)
    d_x = dev(torch_cuda, x)
    xq = torch_cuda.empty(n, dtype=torch_cuda.int8, device="cuda")
    xs = torch_cuda.empty(n // group, dtype=torch_cuda.float32, device="cuda")
    abi.call("l2q_quantize_act", d_x.data_ptr(), n, group, xq.data_ptr(), xs.data_ptr(), stream(torch_cuda))
    torch_cuda.cuda.synchronize()
    np.testing.assert_array_equal(xq.cpu().numpy(), xq_ref)
    np.testing.assert_array_equal(xs.cpu().numpy(), xs_ref)


def near_tie_inputs(n, group, seed):
    """Inputs within a few ulps of (k + 1/2) * s for the group's own scale s:
    the cases where the division-free quantizer must fall back to x / s."""
    rng = np.random.default_rng(seed)
    ng = n // group
    amax = (np.abs(rng.standard_normal(ng)) * 10.0 ** rng.integers(-4, 3, ng)).astype(np.float32) + np.float32(1e-3)
    s = (amax / np.float32(127)).astype(np.float32)
    k = rng.integers(-127, 127, n).astype(np.float32) + np.float32(0.5)
    x = (k * np.repeat(s, group)).astype(np.float32)
    for _ in range(3):
        step = rng.integers(-1, 2, n)
        x = np.where(step > 0, np.nextafter(x, np.float32(np.inf)),
                     np.where(step < 0, np.nextafter(x, np.float32(-np.inf)), x)).astype(np.float32)
    x = np.clip(x, -np.repeat(amax, group), np.repeat(amax, group)).astype(np.float32)
    x[::group] = amax * np.where(rng.random(ng) < 0.5, 1, -1).astype(np.float32)   # pins each group's amax
    return x


@pytest.mark.parametrize("group", [32, 64])
def test_quantize_act_extreme_scales(gpu_lib, torch_cuda, group):
    """Group maxima from denormal to near FLT_MAX: the scale amax/127 (an
    FMA-corrected product on the GPU) and the quantized values must match the
    reference's division bit for bit, also where the scale is denormal."""
    rng = np.random.default_rng(11)
    ng = 512
    n = ng * group
    exps = rng.uniform(-44, 38.5, ng)
    amax = (10.0 ** exps).astype(np.float32)
    amax[:4] = np.array([1e-45, 3e-44, 1e-40, 3.4e38], dtype=np.float32)
    x = (rng.uniform(-1, 1, n).astype(np.float32) * np.repeat(amax, group)).astype(np.float32)
    x[::group] = amax
    xq_ref, xs_ref, _ = O.quantize_act(x, group)
    d_x = dev(torch_cuda, x)
    xq = torch_cuda.empty(n, dtype=torch_cuda.int8, device="cuda")
    xs = torch_cuda.empty(ng, dtype=torch_cuda.float32, device="cuda")
    abi.call("l2q_quantize_act", d_x.data_ptr(), n, group, xq.data_ptr(), xs.data_ptr(), stream(torch_cuda))
    torch_cuda.cuda.synchronize()
    np.testing.assert_array_equal(xs.cpu().numpy(), xs_ref)
    np.testing.assert_array_equal(xq.cpu().numpy(), xq_ref)


@pytest.mark.parametrize("group", [32, 64])
def test_quantize_act_near_ties(gpu_lib, torch_cuda, group):
    n = 1 << 16
    x = near_tie_inputs(n, group, 3)
    xq_ref, xs_ref, _ = O.quantize_act(x, group)
    d_x = dev(torch_cuda, x)
    xq = torch_cuda.empty(n, dtype=torch_cuda.int8, device="cuda")
    xs = torch_cuda.empty(n // group, dtype=torch_cuda.float32, device="cuda")
    abi.call("l2q_quantize_act", d_x.data_ptr(), n, group, xq.data_ptr(), xs.data_ptr(), stream(torch_cuda))
    torch_cuda.cuda.synchronize()
    np.testing.assert_array_equal(xs.cpu().numpy(), xs_ref)
    np.testing.assert_array_equal(xq.cpu().numpy(), xq_ref)


@pytest.mark.parametrize("group", [32, 64])
@pytest.mark.parametrize("n", [288, 768, 4096, 4128])
def test_rmsnorm_quant(gpu_lib, torch_cuda, group, n):
    if n % group:
        pytest.skip("group does not divide n")
    x = host.gauss(n, 5, 1, 1.0)
    r = host.gauss(n, 5, 2, 0.5)
    w = 1.0 + host.gauss(n, 5, 3, 0.1)
    v = (x + r).astype(np.float32)
    o_ref = O.rmsnorm(v, w)
    xq_ref, xs_ref, _ = O.quantize_act(o_ref, group)
    t = torch_cuda
    d_x, d_r, d_w = dev(t, x), dev(t, r), dev(t, w)
    xout = t.empty(n, dtype=t.float32, device="cuda")
    xq = t.empty(n, dtype=t.int8, device="cuda")
    xs = t.empty(n // group, dtype=t.float32, device="cuda")
    abi.call("l2q_rmsnorm_quant", d_x.data_ptr(), d_r.data_ptr(), xout.data_ptr(), d_w.data_ptr(), n, group,
             xq.data_ptr(), xs.data_ptr(), stream(t))
    t.cuda.synchronize()
    np.testing.assert_array_equal(xout.cpu().numpy(), v)          # the residual add is one rounding
    np.testing.assert_array_equal(xq.cpu().numpy(), xq_ref)
    np.testing.assert_array_equal(xs.cpu().numpy(), xs_ref)


@pytest.mark.parametrize("scale", [1e-30, 1e-21, 1e-3, 1e3, 1e18, 1e20])
def test_rmsnorm_quant_extreme_magnitudes(gpu_lib, torch_cuda, scale):
    """Residual streams whose squares underflow into denormals or whose sum of
    squares overflows to inf (inv = 0), with group maxima spread over several
    decades: the fused residual add, RMSNorm and quantize must still equal
    the reference bit for bit."""
    n, group = 4096, 64
    rng = np.random.default_rng(21)
    spread = (10.0 ** rng.uniform(-6, 0, n // group)).astype(np.float32)
    x = (host.gauss(n, 9, 1, 1.0) * np.float32(scale) * np.repeat(spread, group)).astype(np.float32)
    r = (host.gauss(n, 9, 2, 0.5) * np.float32(scale)).astype(np.float32)
    w = 1.0 + host.gauss(n, 9, 3, 0.1)
    v = (x + r).astype(np.float32)
    o_ref = O.rmsnorm(v, w)
    xq_ref, xs_ref, _ = O.quantize_act(o_ref, group)
    t = torch_cuda
    d_x, d_r, d_w = dev(t, x), dev(t, r), dev(t, w)
    xout = t.empty(n, dtype=t.float32, device="cuda")
    xq = t.empty(n, dtype=t.int8, device="cuda")
    xs = t.empty(n // group, dtype=t.float32, device="cuda")
    abi.call("l2q_rmsnorm_quant", d_x.data_ptr(), d_r.data_ptr(), xout.data_ptr(), d_w.data_ptr(), n, group,
             xq.data_ptr(), xs.data_ptr(), stream(t))
    t.cuda.synchronize()
    np.testing.assert_array_equal(xout.cpu().numpy(), v)
    np.testing.assert_array_equal(xs.cpu().numpy(), xs_ref)
    np.testing.assert_array_equal(xq.cpu().numpy(), xq_ref)


@pytest.mark.parametrize("group", [32, 64])
@pytest.mark.parametrize("n", [768, 11008])
def test_swiglu_quant(gpu_lib, torch_cuda, group, n):
    if n % group:
        pytest.skip("group does not divide n")
    h = host.gauss(n, 8, 1, 2.0)
    h2 = host.gauss(n, 8, 2, 2.0)
    g_ref = O.swiglu(h, h2)
    xq_ref, xs_ref, _ = O.quantize_act(g_ref, group)
    t = torch_cuda
    d_h, d_h2 = dev(t, h), dev(t, h2)
    gout = t.empty(n, dtype=t.float32, device="cuda")
    xq = t.empty(n, dtype=t.int8, device="cuda")
    xs = t.empty(n // group, dtype=t.float32, device="cuda")
    abi.call("l2q_swiglu_quant", d_h.data_ptr(), d_h2.data_ptr(), n, group, xq.data_ptr(), xs.data_ptr(),
             gout.data_ptr(), stream(t))
    t.cuda.synchronize()
    np.testing.assert_array_equal(gout.cpu().numpy(), g_ref)
    np.testing.assert_array_equal(xq.cpu().numpy(), xq_ref)
    np.testing.assert_array_equal(xs.cpu().numpy(), xs_ref)


@pytest.mark.parametrize("scale", [1e-30, 1e-3, 30.0, 1e4, 1e15])
def test_swiglu_quant_extreme_magnitudes(gpu_lib, torch_cuda, scale):
    """SwiGLU over gate values where expf underflows, saturates or overflows
    (silu -> 0 or h), tiny and huge up-projections, group maxima over several
    decades: bit for bit against the reference."""
    n, group = 11008, 64
    rng = np.random.default_rng(23)
    spread = (10.0 ** rng.uniform(-5, 0, n // group)).astype(np.float32)
    h = (host.gauss(n, 10, 1, 1.0) * np.float32(scale)).astype(np.float32)
    h2 = (host.gauss(n, 10, 2, 1.0) * np.float32(scale) * np.repeat(spread, group)).astype(np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        g_ref = O.swiglu(h, h2)
    xq_ref, xs_ref, _ = O.quantize_act(g_ref, group)
    t = torch_cuda
    d_h, d_h2 = dev(t, h), dev(t, h2)
    gout = t.empty(n, dtype=t.float32, device="cuda")
    xq = t.empty(n, dtype=t.int8, device="cuda")
    xs = t.empty(n // group, dtype=t.float32, device="cuda")
    abi.call("l2q_swiglu_quant", d_h.data_ptr(), d_h2.data_ptr(), n, group, xq.data_ptr(), xs.data_ptr(),
             gout.data_ptr(), stream(t))
    t.cuda.synchronize()
    np.testing.assert_array_equal(gout.cpu().numpy(), g_ref)
    np.testing.assert_array_equal(xs.cpu().numpy(), xs_ref)
    np.testing.assert_array_equal(xq.cpu().numpy(), xq_ref)


def attention_case(t, n_heads, n_kv, hs, max_t, pos, seed, entry="l2q_attention"):
    """Fill caches for positions < pos, then RoPE + append at pos and attend."""
    kv_dim = n_kv * hs
    kc = host.gauss(n_kv * max_t * hs, seed, 1, 1.0).reshape(n_kv, max_t, hs)
    vc = host.gauss(n_kv * max_t * hs, seed, 2, 1.0).reshape(n_kv, max_t, hs)
    q = host.gauss(n_heads * hs, seed, 3, 1.0)
    k = host.gauss(kv_dim, seed, 4, 1.0)
    v = host.gauss(kv_dim, seed, 5, 1.0)
    # oracle: rope then append then attend
    qr, kr = O.rope(q, k, pos, hs)
    kc_ref, vc_ref = kc.copy(), vc.copy()
    kc_ref[:, pos, :] = kr.reshape(n_kv, hs)
    vc_ref[:, pos, :] = v.reshape(n_kv, hs)
    out_ref = O.attention(qr, kc_ref, vc_ref, pos, n_heads, n_kv, hs)
    # GPU
    rope = np.empty(max_t * hs, dtype=np.float32)
    abi.lib().l2q_rope_table(rope.ctypes.data, max_t, hs)
    d_q, d_k, d_v = dev(t, q), dev(t, k), dev(t, v)
    d_kc, d_vc, d_rope = dev(t, kc), dev(t, vc), dev(t, rope)
    out = t.empty(n_heads * hs, dtype=t.float32, device="cuda")
    abi.call("l2q_rope_kv_append", d_q.data_ptr(), d_k.data_ptr(), d_v.data_ptr(), d_kc.data_ptr(),
             d_vc.data_ptr(), d_rope.data_ptr(), pos, n_heads, n_kv, hs, max_t, stream(t))
    abi.call(entry, d_q.data_ptr(), d_kc.data_ptr(), d_vc.data_ptr(), out.data_ptr(), pos, n_heads, n_kv,
             hs, max_t, stream(t))
    t.cuda.synchronize()
    return (qr, kc_ref, vc_ref, out_ref), (d_q.cpu().numpy(), d_kc.cpu().numpy(), d_vc.cpu().numpy(),
                                           out.cpu().numpy())


@pytest.mark.parametrize("ctx", [1, 2, 63, 64, 65, 256, 1024, 2048, 4096])
def test_rope_append_attention_c4(gpu_lib, torch_cuda, ctx):
    """c4: 32 heads x 128, fp32 cache of 4096 positions, RoPE theta 1e4."""
    print(f"attention ctx={ctx}", flush=True)
    ref, got = attention_case(torch_cuda, 32, 32, 128, 4096, ctx - 1, 40 + ctx)
    np.testing.assert_array_equal(got[0], ref[0])     # rotated q
    np.testing.assert_array_equal(got[1], ref[1])     # K cache incl. the appended row
    np.testing.assert_array_equal(got[2], ref[2])     # V cache
    np.testing.assert_array_equal(got[3], ref[3])     # output, bit-exact


@pytest.mark.parametrize("ctx", [1, 65, 256, 1024, 2048, 4096])
def test_attention_split_c4(gpu_lib, torch_cuda, ctx):
    """The split-context variant: 1e-5 relative (c4 tolerance)."""
    ref, got = attention_case(torch_cuda, 32, 32, 128, 4096, ctx - 1, 40 + ctx, "l2q_attention_split")
    assert_close(got[3], ref[3], 1e-5, what=f"split attention ctx={ctx}")


@pytest.mark.parametrize("n_heads,n_kv,hs,max_t,pos", [
    (6, 6, 48, 256, 0), (6, 6, 48, 256, 100), (6, 6, 48, 256, 255),   # c1 heads
    (8, 2, 64, 512, 300),                                              # grouped-query heads
])
def test_attention_other_heads(gpu_lib, torch_cuda, n_heads, n_kv, hs, max_t, pos):
    ref, got = attention_case(torch_cuda, n_heads, n_kv, hs, max_t, pos, 7)
    np.testing.assert_array_equal(got[0], ref[0])
    np.testing.assert_array_equal(got[1], ref[1])
    np.testing.assert_array_equal(got[3], ref[3])


@pytest.mark.parametrize("n_heads,n_kv,hs,max_t,ctx", [
    (32, 32, 128, 4096, 1), (32, 32, 128, 4096, 65), (32, 32, 128, 4096, 513), (32, 32, 128, 4096, 769),
    (32, 32, 128, 4096, 4096), (6, 6, 48, 256, 1), (6, 6, 48, 256, 256), (8, 2, 64, 512, 300),
])
def test_attention_forms_and_k_layouts(gpu_lib, torch_cuda, n_heads, n_kv, hs, max_t, ctx):
    """The single-kernel and two-kernel forms, over the row-major and the
    engine's column-interleaved K layout ([n_kv][hs/4][max_t][4]), all give
    the oracle's bits (runq.c:367-391)."""
    t = torch_cuda
    print(f"attention forms heads={n_heads}/{n_kv} hs={hs} ctx={ctx}", flush=True)
    pos = ctx - 1
    kc = host.gauss(n_kv * max_t * hs, ctx, 1, 1.0).reshape(n_kv, max_t, hs)
    vc = host.gauss(n_kv * max_t * hs, ctx, 2, 1.0).reshape(n_kv, max_t, hs)
    q = host.gauss(n_heads * hs, ctx, 3, 1.0)
    ref = O.attention(q, kc, vc, pos, n_heads, n_kv, hs)
    kil = np.ascontiguousarray(kc.reshape(n_kv, max_t, hs // 4, 4).transpose(0, 2, 1, 3))
    d_q, d_v = dev(t, q), dev(t, vc)
    out = t.empty(n_heads * hs, dtype=t.float32, device="cuda")
    for layout, kd in ((0, dev(t, kc)), (abi.L2Q_ATTN_K_INTERLEAVED, dev(t, kil))):
        for form in (0, abi.L2Q_ATTN_ONE_KERNEL, abi.L2Q_ATTN_TWO_KERNELS):
            out.fill_(np.nan)
            abi.call("l2q_attention_ex", d_q.data_ptr(), kd.data_ptr(), d_v.data_ptr(), out.data_ptr(), pos, n_heads,
                     n_kv, hs, max_t, layout | form, stream(t))
            t.cuda.synchronize()
            np.testing.assert_array_equal(out.cpu().numpy(), ref, err_msg=f"layout {layout} form {form}")


@pytest.mark.parametrize("n_heads,n_kv,hs,max_t,ctx,scale", [
    (32, 32, 128, 4096, 1, 1.0), (32, 32, 128, 4096, 64, 1.0), (32, 32, 128, 4096, 65, 1.0),
    (32, 32, 128, 4096, 1024, 1.0), (32, 32, 128, 4096, 1025, 1.0), (32, 32, 128, 4096, 2049, 1.0),
    (32, 32, 128, 4096, 4096, 1.0), (6, 6, 48, 256, 1, 1.0), (6, 6, 48, 256, 256, 1.0),
    (8, 2, 64, 512, 300, 1.0), (32, 8, 128, 4096, 3000, 1.0),
    (32, 32, 128, 4096, 700, 1e-30), (32, 32, 128, 4096, 700, 1e15), (32, 32, 128, 4096, 1500, 30.0),
])
def test_attention_split_context_tolerance(gpu_lib, torch_cuda, n_heads, n_kv, hs, max_t, ctx, scale):
    """L2Q_ATTN_SPLIT_CONTEXT (the engine's tolerance-mode attention: the
    context split over ~2 workgroups per CU, per-split softmax partials
    merged in split order by the last workgroup of each head) in both K
    layouts: within 1e-5 of the oracle's exact order (elementwise, floor at
    the output's RMS), at contexts of one to several 64-position score blocks
    per split, GQA, and score magnitudes from ~0 to ~1e30."""
    t = torch_cuda
    print(f"attention split-context heads={n_heads}/{n_kv} hs={hs} ctx={ctx} scale={scale}", flush=True)
    pos = ctx - 1
    sc = np.float32(scale)
    kc = (host.gauss(n_kv * max_t * hs, ctx, 1, 1.0) * sc).astype(np.float32).reshape(n_kv, max_t, hs)
    vc = host.gauss(n_kv * max_t * hs, ctx, 2, 1.0).reshape(n_kv, max_t, hs)
    q = (host.gauss(n_heads * hs, ctx, 3, 1.0) * sc).astype(np.float32)
    ref = O.attention(q, kc, vc, pos, n_heads, n_kv, hs)
    kil = np.ascontiguousarray(kc.reshape(n_kv, max_t, hs // 4, 4).transpose(0, 2, 1, 3))
    d_q, d_v = dev(t, q), dev(t, vc)
    out = t.empty(n_heads * hs, dtype=t.float32, device="cuda")
    for layout, kd in ((0, dev(t, kc)), (abi.L2Q_ATTN_K_INTERLEAVED, dev(t, kil))):
        for rep in range(2):   # the second call finds the counters the first left zeroed
            out.fill_(np.nan)
            abi.call("l2q_attention_ex", d_q.data_ptr(), kd.data_ptr(), d_v.data_ptr(), out.data_ptr(), pos, n_heads,
                     n_kv, hs, max_t, layout | abi.L2Q_ATTN_SPLIT_CONTEXT, stream(t))
            t.cuda.synchronize()
            assert_close(out.cpu().numpy(), ref, 1e-5, what=f"layout {layout} call {rep}")


@pytest.mark.parametrize("scale", [1e-30, 1e-6, 30.0, 1e6, 1e15])
@pytest.mark.parametrize("ctx", [65, 700])
def test_attention_forms_extreme_magnitudes(gpu_lib, torch_cuda, scale, ctx):
    """Scores from ~0 (a uniform softmax, values that underflow in the
    products) to ~1e30 (a softmax that collapses onto one position, exp
    underflowing to 0 for the rest), in every form and K layout: the
    oracle's bits."""
    t = torch_cuda
    n_heads = n_kv = 8
    hs, max_t = 128, 1024
    pos = ctx - 1
    kc = (host.gauss(n_kv * max_t * hs, ctx, 1, 1.0) * np.float32(scale)).astype(np.float32).reshape(n_kv, max_t, hs)
    vc = host.gauss(n_kv * max_t * hs, ctx, 2, 1.0).reshape(n_kv, max_t, hs)
    q = (host.gauss(n_heads * hs, ctx, 3, 1.0) * np.float32(scale)).astype(np.float32)
    ref = O.attention(q, kc, vc, pos, n_heads, n_kv, hs)
    kil = np.ascontiguousarray(kc.reshape(n_kv, max_t, hs // 4, 4).transpose(0, 2, 1, 3))
    d_q, d_v = dev(t, q), dev(t, vc)
    out = t.empty(n_heads * hs, dtype=t.float32, device="cuda")
    for layout, kd in ((0, dev(t, kc)), (abi.L2Q_ATTN_K_INTERLEAVED, dev(t, kil))):
        for form in (abi.L2Q_ATTN_ONE_KERNEL, abi.L2Q_ATTN_TWO_KERNELS):
            out.fill_(np.nan)
            abi.call("l2q_attention_ex", d_q.data_ptr(), kd.data_ptr(), d_v.data_ptr(), out.data_ptr(), pos, n_heads,
                     n_kv, hs, max_t, layout | form, stream(t))
            t.cuda.synchronize()
            np.testing.assert_array_equal(out.cpu().numpy(), ref, err_msg=f"layout {layout} form {form}")


def test_expf_identical_to_host_on_every_input(gpu_lib, torch_cuda):
    """The device exp used by softmax and SwiGLU equals the host C library's
    expf on all 2^32 float bit patterns (NaNs compared as NaN)."""
    t = torch_cuda
    chunk = 1 << 27
    ybuf = t.empty(chunk, dtype=t.float32, device="cuda")
    for c in range((1 << 32) // chunk):
        bits = np.arange(c * chunk, (c + 1) * chunk, dtype=np.uint64).astype(np.uint32)
        x = bits.view(np.float32)
        d_x = dev(t, x)
        abi.call("l2q_expf", d_x.data_ptr(), ybuf.data_ptr(), chunk, stream(t))
        t.cuda.synchronize()
        y = ybuf.cpu().numpy()
        ref = O.expf_host(x)
        same = (y.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(y) & np.isnan(ref))
        assert same.all(), f"chunk {c}: {int((~same).sum())} mismatches, first x={x[~same][0]!r}"


@pytest.mark.parametrize("n", [1, 3, 4, 5, 1000, 32000, 32003, 40000])
def test_argmax_first_index(gpu_lib, torch_cuda, n):
    """Device argmax = the first index of the maximum (runq.c:578-585):
    random values, ties planted before and after the maximum's first
    occurrence, an all-equal vector, and a maximum in the scalar tail."""
    t = torch_cuda
    rng = np.random.default_rng(n)
    out = t.zeros(1, dtype=t.int32, device="cuda")
    cases = [rng.standard_normal(n).astype(np.float32), np.full(n, -2.5, np.float32)]
    v = rng.standard_normal(n).astype(np.float32)
    v[rng.integers(0, n, size=min(n, 3))] = 9.0     # several copies of the maximum
    cases.append(v)
    v = rng.standard_normal(n).astype(np.float32)
    v[-1] = 7.0                                    # in the tail when n % 4
    cases.append(v)
    # NaN and -inf, where the reference's scan (start from v[0], take
    # v[i] > max) differs from numpy's argmax: NaNs are skipped, a NaN at
    # index 0 answers 0, an all -inf vector answers 0
    v = rng.standard_normal(n).astype(np.float32)
    v[rng.integers(0, n, size=min(n, 5))] = np.nan
    cases.append(v)
    v = rng.standard_normal(n).astype(np.float32)
    v[0] = np.nan
    cases.append(v)
    cases.append(np.full(n, -np.inf, np.float32))
    cases.append(np.full(n, np.nan, np.float32))
    for v in cases:
        d_v = dev(t, v)
        abi.call("l2q_argmax", d_v.data_ptr(), n, out.data_ptr(), stream(t))
        t.cuda.synchronize()
        assert int(out.item()) == O.argmax(v), (n, v[:8])


def test_unbias(gpu_lib, torch_cuda):
    t = torch_cuda
    src = np.arange(1000, dtype=np.int64).astype(np.uint8)
    d_src = dev(t, src)
    dst = t.empty(1000, dtype=t.int8, device="cuda")
    abi.call("l2q_unbias_q8", d_src.data_ptr(), dst.data_ptr(), 1000, stream(t))
    t.cuda.synchronize()
    np.testing.assert_array_equal(dst.cpu().numpy(), (src.astype(np.int16) - 128).astype(np.int8))


def test_bad_shapes_raise(gpu_lib, torch_cuda):
    t = torch_cuda
    buf = t.zeros(1 << 16, dtype=t.uint8, device="cuda")
    p = buf.data_ptr()
    with pytest.raises(abi.L2QError):
        abi.call("l2q_gemv_q4", p, p, p, p, p, 16, 100, 64, None, None)       # cols % group
    with pytest.raises(abi.L2QError):
        abi.call("l2q_gemv_q8", p, p + 1, p, p, p, 16, 4096, 64, None, None)  # misaligned activations
    with pytest.raises(abi.L2QError):
        abi.call("l2q_attention", p, p, p, p, 10, 4, 4, 128, 8, None)         # pos >= max_t
    with pytest.raises(abi.L2QError):
        abi.call("l2q_attention_ex", p, p, p, p, 1, 4, 4, 96, 8, abi.L2Q_ATTN_ONE_KERNEL, None)   # no 96 form
    with pytest.raises(abi.L2QError):
        abi.call("l2q_attention_ex", p, p, p, p, 1, 4, 4, 128, 8, 6, None)     # both forms
    with pytest.raises(abi.L2QError):
        abi.call("l2q_attention_ex", p, p, p, p, 1, 4, 4, 128, 8, 16, None)    # unknown flag
    with pytest.raises(abi.L2QError):
        abi.call("l2q_attention_ex", p, p, p, p, 1, 4, 4, 128, 8, 10, None)    # split context + one kernel
    with pytest.raises(abi.L2QError):
        abi.call("l2q_attention_ex", p, p, p, p, 1, 4, 4, 96, 8, abi.L2Q_ATTN_SPLIT_CONTEXT, None)  # no 96 form

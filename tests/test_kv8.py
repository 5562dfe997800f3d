"""int8 KV cache (the reference's INT8_KV build, v5-cuda-fused/run.cu:41-48,
204-249, 350-410).

Oracle pins (CPU): orc_kv_quant against its closed form (amax/127, rint,
clamp; zero rows; the extreme element maps to +-127), and
orc_attention_kv8 (evaluated in double) against the bit-exact fp32
attention oracle (runq.c:367-391) run on the dequantized caches -- an
independent path, so a wrong scale index, head mapping or position stride
fails it; the oracle's restatement in the GPU kernels' float order agrees
with the double one.  GPU parity: l2q_kv8_append is bit-exact (int8 rows
and scales, RoPE included); l2q_attention_kv8 is within 2e-5 relative
(floor: output RMS) of the double-precision oracle at the c4 shapes and
bit-exact against the ordered restatement; its split-context form
(l2q_attention_kv8_ex with L2Q_ATTN_SPLIT_CONTEXT, the engine's) is within
the same 2e-5 and bit-exact against orc_attention_kv8_split, the oracle's
restatement of its order; the engine with L2Q_ENGINE_KV_INT8 reproduces the
oracle's int8-KV forward (in the split order, with the engine's split
count) bit for bit.
"""
import numpy as np
import pytest

from conftest import assert_close, rel_err
from llama2q import abi, host
import oracle_py as O


def kv_quant_closed_form(row):
    row = np.asarray(row, dtype=np.float32)
    s = np.float32(np.abs(row).max() / np.float32(127.0))
    if s == 0.0:
        s = np.float32(1e-8)
    q = np.clip(np.rint(row / s), -127, 127).astype(np.int8)
    return q, s


@pytest.mark.parametrize("hs", [48, 128, 256])
def test_kv_quant_closed_form(hs):
    for seed in range(6):
        row = host.gauss(hs, seed, 9, 0.5 + seed)
        if seed == 1:
            row[:] = 0.0
        if seed == 2:
            row[5] = -3.0 * np.abs(row).max()
        q, s = O.kv_quant(row)
        eq, es = kv_quant_closed_form(row)
        assert s == es
        np.testing.assert_array_equal(q, eq)
        if seed != 1:
            assert np.abs(q).max() == 127
        else:
            assert s == np.float32(1e-8) and not q.any()


def random_kv8(n_kv, max_t, hs, seed):
    rng = np.random.default_rng(seed)
    k8 = rng.integers(-127, 128, size=(n_kv, max_t, hs), dtype=np.int8)
    v8 = rng.integers(-127, 128, size=(n_kv, max_t, hs), dtype=np.int8)
    ks = (rng.random((n_kv, max_t), dtype=np.float32) * 0.02 + 1e-3).astype(np.float32)
    vs = (rng.random((n_kv, max_t), dtype=np.float32) * 0.02 + 1e-3).astype(np.float32)
    return k8, v8, ks, vs


@pytest.mark.parametrize("n_heads,n_kv,hs,pos", [(6, 6, 48, 0), (6, 6, 48, 70), (8, 2, 64, 130), (4, 4, 128, 255)])
def test_attention_kv8_oracle_equals_fp32_attention_on_dequantized(n_heads, n_kv, hs, pos):
    max_t = pos + 3
    k8, v8, ks, vs = random_kv8(n_kv, max_t, hs, pos + hs)
    q = host.gauss(n_heads * hs, pos, 3, 1.0)
    got = O.attention_kv8(q, k8, v8, ks, vs, pos, n_heads, n_kv, hs)
    kd = (k8.astype(np.float32) * ks[:, :, None]).astype(np.float32)
    vd = (v8.astype(np.float32) * vs[:, :, None]).astype(np.float32)
    ref = O.attention(q, kd, vd, pos, n_heads, n_kv, hs)
    assert_close(got, ref, 2e-5, what="kv8 oracle vs fp32 attention")
    # the GPU-order float restatement agrees with the double one
    ordered = O.attention_kv8(q, k8, v8, ks, vs, pos, n_heads, n_kv, hs, ordered=True)
    assert_close(ordered, got, 2e-5, what="kv8 ordered vs double")


@pytest.mark.parametrize("n_heads,n_kv,hs,pos,S", [
    (6, 6, 48, 0, 64), (6, 6, 48, 70, 64), (8, 2, 64, 130, 16), (4, 4, 128, 255, 1), (4, 4, 128, 255, 2),
    (4, 4, 128, 600, 8), (32, 8, 128, 1000, 16), (2, 2, 128, 4095, 16)])
def test_attention_kv8_split_oracle_equals_double(n_heads, n_kv, hs, pos, S):
    """The split restatement (the split kernel's float order: per-split
    softmax partials merged in split order) is within 2e-5 of the double
    oracle for one split, splits of one position, empty splits (S > n),
    GQA and 4096 positions; the split order also differs from the
    one-workgroup order's bits, so the two restatements are distinct."""
    max_t = pos + 3
    k8, v8, ks, vs = random_kv8(n_kv, max_t, hs, pos + hs + S)
    q = host.gauss(n_heads * hs, pos, 4, 1.0)
    ref = O.attention_kv8(q, k8, v8, ks, vs, pos, n_heads, n_kv, hs)
    got = O.attention_kv8(q, k8, v8, ks, vs, pos, n_heads, n_kv, hs, splits=S)
    assert_close(got, ref, 2e-5, what=f"kv8 split S={S} vs double")


def test_attention_kv8_split_oracle_scale_invariances():
    """Closed-form checks the double pin cannot separate: scaling every V
    scale by 2 doubles the output exactly (powers of two commute with every
    rounding), and adding a constant to every score (a K row equal for all
    positions scaled per position is not constant, so use q = 0) gives the
    uniform average of the dequantized V rows."""
    n_heads = n_kv = 2
    hs, pos, S = 64, 300, 16
    k8, v8, ks, vs = random_kv8(n_kv, pos + 1, hs, 5)
    q = host.gauss(n_heads * hs, 5, 4, 1.0)
    a = O.attention_kv8(q, k8, v8, ks, vs, pos, n_heads, n_kv, hs, splits=S)
    b = O.attention_kv8(q, k8, v8, ks, (vs * np.float32(2.0)).astype(np.float32), pos, n_heads, n_kv, hs, splits=S)
    np.testing.assert_array_equal(b, a * np.float32(2.0))
    z = O.attention_kv8(np.zeros_like(q), k8, v8, ks, vs, pos, n_heads, n_kv, hs, splits=S)
    vd = (v8.astype(np.float64) * vs[:, :, None].astype(np.float64))[:, :pos + 1]
    want = np.repeat(vd.mean(axis=1), n_heads // n_kv, axis=0).reshape(-1)
    assert_close(z, want.astype(np.float32), 1e-5, what="uniform softmax")


def test_oracle_kv8_forward_tracks_fp32_forward():
    """int8 K/V costs ~0.4% per vector (v5-cuda-fused/run.cu:41-45): the
    logits of the int8-KV oracle stay close to the fp32-KV oracle's."""
    ck = host.synth_checkpoint(host.config_15m(), 8, 32, seed=77)
    a = O.Oracle(ck.cfg.as_list(), ck.weights, 8, 32, max_t=64)
    b = O.Oracle(ck.cfg.as_list(), ck.weights, 8, 32, max_t=64, kv8=True)
    token = 9
    for pos in range(24):
        la, lb = a.forward(token, pos), b.forward(token, pos)
        assert rel_err(lb, la) < 0.05, pos
        if pos == 0:   # one position: softmax weight 1, out = dequantized v
            assert rel_err(lb, la) < 0.02
        token = int(np.argmax(la))


# --------------------------------------------------------------------------- GPU


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def stream(torch):
    return torch.cuda.current_stream().cuda_stream


@pytest.mark.gpu
@pytest.mark.parametrize("n_kv,hs", [(6, 48), (32, 128), (2, 256)])
def test_gpu_kv8_append_bit_exact(gpu_lib, torch_cuda, n_kv, hs):
    t = torch_cuda
    max_t = 96
    rope = np.empty(max_t * hs, dtype=np.float32)
    abi.lib().l2q_rope_table(rope.ctypes.data, max_t, hs)
    d_rope = dev(t, rope)
    k8 = t.zeros(n_kv * max_t * hs, dtype=t.int8, device="cuda")
    v8 = t.zeros_like(k8)
    ks = t.zeros(n_kv * max_t, dtype=t.float32, device="cuda")
    vs = t.zeros_like(ks)
    ek8 = np.zeros((n_kv, max_t, hs), np.int8)
    ev8 = np.zeros_like(ek8)
    eks = np.zeros((n_kv, max_t), np.float32)
    evs = np.zeros_like(eks)
    for pos in (0, 1, 17, 95):
        print(f"kv8 append n_kv={n_kv} hs={hs} pos={pos}", flush=True)
        k = host.gauss(n_kv * hs, pos, 4, 1.0 + pos)
        v = host.gauss(n_kv * hs, pos, 5, 2.0)
        if pos == 17:
            v[:hs] = 0.0            # a zero row: scale 1e-8
        d_k, d_v = dev(t, k), dev(t, v)
        abi.call("l2q_kv8_append", d_k.data_ptr(), d_v.data_ptr(), k8.data_ptr(), v8.data_ptr(), ks.data_ptr(),
                 vs.data_ptr(), d_rope.data_ptr(), pos, n_kv, hs, max_t, stream(t))
        _, kr = O.rope(np.zeros(n_kv * hs, np.float32), k, pos, hs)
        for g in range(n_kv):
            ek8[g, pos], eks[g, pos] = O.kv_quant(kr[g * hs:(g + 1) * hs])
            ev8[g, pos], evs[g, pos] = O.kv_quant(v[g * hs:(g + 1) * hs])
    t.cuda.synchronize()
    np.testing.assert_array_equal(k8.cpu().numpy().reshape(ek8.shape), ek8)
    np.testing.assert_array_equal(v8.cpu().numpy().reshape(ev8.shape), ev8)
    np.testing.assert_array_equal(ks.cpu().numpy().reshape(eks.shape), eks)
    np.testing.assert_array_equal(vs.cpu().numpy().reshape(evs.shape), evs)


@pytest.mark.gpu
@pytest.mark.parametrize("scale", [1e-44, 1e-40, 1e-37, 1e30])
def test_gpu_kv8_append_extreme_magnitudes(gpu_lib, torch_cuda, scale):
    """k and v rows from denormal (scales amax/127 of a few bits, where the
    clamp to +-127 binds) to 1e30, RoPE applied to k: bit for bit."""
    t = torch_cuda
    n_kv, hs, max_t = 4, 128, 16
    rope = np.empty(max_t * hs, dtype=np.float32)
    abi.lib().l2q_rope_table(rope.ctypes.data, max_t, hs)
    d_rope = dev(t, rope)
    k8 = t.zeros(n_kv * max_t * hs, dtype=t.int8, device="cuda")
    v8 = t.zeros_like(k8)
    ks = t.zeros(n_kv * max_t, dtype=t.float32, device="cuda")
    vs = t.zeros_like(ks)
    for pos in (0, 5):
        k = (host.gauss(n_kv * hs, pos, 6, 1.0) * np.float32(scale)).astype(np.float32)
        v = (host.gauss(n_kv * hs, pos, 7, 1.0) * np.float32(scale)).astype(np.float32)
        d_k, d_v = dev(t, k), dev(t, v)
        abi.call("l2q_kv8_append", d_k.data_ptr(), d_v.data_ptr(), k8.data_ptr(), v8.data_ptr(), ks.data_ptr(),
                 vs.data_ptr(), d_rope.data_ptr(), pos, n_kv, hs, max_t, stream(t))
        t.cuda.synchronize()
        _, kr = O.rope(np.zeros(n_kv * hs, np.float32), k, pos, hs)
        g8 = k8.cpu().numpy().reshape(n_kv, max_t, hs)
        h8 = v8.cpu().numpy().reshape(n_kv, max_t, hs)
        gks = ks.cpu().numpy().reshape(n_kv, max_t)
        gvs = vs.cpu().numpy().reshape(n_kv, max_t)
        for g in range(n_kv):
            eq, es = O.kv_quant(kr[g * hs:(g + 1) * hs])
            np.testing.assert_array_equal(g8[g, pos], eq)
            assert gks[g, pos] == es
            eq, es = O.kv_quant(v[g * hs:(g + 1) * hs])
            np.testing.assert_array_equal(h8[g, pos], eq)
            assert gvs[g, pos] == es


@pytest.mark.gpu
@pytest.mark.parametrize("n_heads,n_kv,hs,max_t,ctx", [(32, 32, 128, 4096, 1), (32, 32, 128, 4096, 64),
                                                      (32, 32, 128, 4096, 256), (32, 32, 128, 4096, 1024),
                                                      (32, 32, 128, 4096, 4096), (6, 6, 48, 256, 200),
                                                      (8, 2, 64, 512, 333)])
def test_gpu_attention_kv8(gpu_lib, torch_cuda, n_heads, n_kv, hs, max_t, ctx):
    """c4 shapes (32 heads x 128, cache of 4096 positions) and GQA."""
    t = torch_cuda
    print(f"attention kv8 heads={n_heads}/{n_kv} hs={hs} ctx={ctx}", flush=True)
    pos = ctx - 1
    k8, v8, ks, vs = random_kv8(n_kv, max_t, hs, ctx + hs)
    q = host.gauss(n_heads * hs, ctx, 3, 1.0)
    ref = O.attention_kv8(q, k8, v8, ks, vs, pos, n_heads, n_kv, hs)
    out = t.empty(n_heads * hs, dtype=t.float32, device="cuda")
    d = [dev(t, a) for a in (q, k8, v8, ks, vs)]
    abi.call("l2q_attention_kv8", *[x.data_ptr() for x in d], out.data_ptr(), pos, n_heads, n_kv, hs, max_t,
             stream(t))
    t.cuda.synchronize()
    got = out.cpu().numpy()
    assert_close(got, ref, 2e-5, what=f"attention kv8 ctx={ctx}")
    # bit for bit against the oracle evaluated in the kernels' float order
    np.testing.assert_array_equal(got, O.attention_kv8(q, k8, v8, ks, vs, pos, n_heads, n_kv, hs, ordered=True))


@pytest.mark.gpu
def flash_splits(n_heads, n, ncu):
    """The library's split count for n positions (about two workgroups per
    CU, at most 256 positions per split, 1..64 splits)."""
    S = max(-(-2 * ncu // n_heads), -(-n // 256))
    return min(max(S, 1), 64)


@pytest.mark.gpu
@pytest.mark.parametrize("n_heads,n_kv,hs,max_t,ctx", [(32, 32, 128, 4096, 1), (32, 32, 128, 4096, 64),
                                                      (32, 32, 128, 4096, 257), (32, 32, 128, 4096, 1024),
                                                      (32, 32, 128, 4096, 4096), (6, 6, 48, 256, 200),
                                                      (8, 2, 64, 512, 333), (32, 8, 128, 8192, 8192),
                                                      (2, 2, 256, 300, 300)])
def test_gpu_attention_kv8_split(gpu_lib, torch_cuda, n_heads, n_kv, hs, max_t, ctx):
    """The split-context form: 2e-5 of the double formula, and bit for bit
    the oracle's restatement of its order (per-split softmax partials, one
    to several 64-position rounds per split, empty splits, GQA, head sizes
    48 to 256, 8192 positions); two calls in a row (the counters the first
    leaves zeroed serve the second)."""
    t = torch_cuda
    print(f"attention kv8 split heads={n_heads}/{n_kv} hs={hs} ctx={ctx}", flush=True)
    pos = ctx - 1
    k8, v8, ks, vs = random_kv8(n_kv, max_t, hs, ctx + hs + 1)
    q = host.gauss(n_heads * hs, ctx, 5, 1.0)
    S = flash_splits(n_heads, ctx, t.cuda.get_device_properties(0).multi_processor_count)
    ref = O.attention_kv8(q, k8, v8, ks, vs, pos, n_heads, n_kv, hs)
    want = O.attention_kv8(q, k8, v8, ks, vs, pos, n_heads, n_kv, hs, splits=S)
    out = t.empty(n_heads * hs, dtype=t.float32, device="cuda")
    d = [dev(t, a) for a in (q, k8, v8, ks, vs)]
    for rep in range(2):
        out.fill_(np.nan)
        abi.call("l2q_attention_kv8_ex", *[x.data_ptr() for x in d], out.data_ptr(), pos, n_heads, n_kv, hs, max_t,
                 abi.L2Q_ATTN_SPLIT_CONTEXT, stream(t))
        t.cuda.synchronize()
        got = out.cpu().numpy()
        assert_close(got, ref, 2e-5, what=f"attention kv8 split ctx={ctx} S={S}")
        np.testing.assert_array_equal(got, want, err_msg=f"call {rep}, S={S}")


@pytest.mark.gpu
def test_gpu_attention_kv8_rejects_bad_shapes(gpu_lib, torch_cuda):
    t = torch_cuda
    buf = t.zeros(1 << 16, dtype=t.float32, device="cuda")
    p = buf.data_ptr()
    for hs, max_t, pos in ((40, 64, 0), (128, 64, 64), (128, 9000, 0)):
        rc = abi.lib().l2q_attention_kv8(p, p, p, p, p, p, pos, 1, 1, hs, max_t, stream(t))
        assert rc == abi.L2Q_ERR_ARG
        rc = abi.lib().l2q_attention_kv8_ex(p, p, p, p, p, p, pos, 1, 1, hs, max_t, abi.L2Q_ATTN_SPLIT_CONTEXT,
                                            stream(t))
        assert rc == abi.L2Q_ERR_ARG
    assert abi.lib().l2q_attention_kv8_ex(p, p, p, p, p, p, 0, 1, 1, 128, 64, 2, stream(t)) == abi.L2Q_ERR_ARG


@pytest.mark.gpu
@pytest.mark.parametrize("shape", ["c1_q8_g32", "7b2_q4_g64", "gqa_hs64_q4_g32", "c1_q8_g32_long"])
def test_gpu_engine_kv8_follows_oracle(gpu_lib, torch_cuda, shape):
    """Engine with the int8 KV cache against the oracle's int8-KV forward
    (attention in the one-workgroup order up to L2Q_KV8_SPLIT_FROM positions
    and in the split order with the engine's split count beyond): logits bit
    for bit at every step of a greedy decode, so the token ids are
    identical; the long case crosses the switch (positions 0..1099)."""
    from llama2q.model import Engine
    if shape == "c1_q8_g32":
        ck = host.synth_checkpoint(host.config_15m(), 8, 32, seed=21)
        steps = 64
    elif shape == "c1_q8_g32_long":   # c1's widths, two layers, a 2048-position context
        cfg = host.make_config(288, 768, 2, 6, 6, 512, 2048)
        ck = host.synth_checkpoint(cfg, 8, 32, seed=25)
        steps = 1100
    elif shape == "gqa_hs64_q4_g32":   # 4 heads over 2 kv heads: the group's first head appends
        cfg = host.make_config(256, 512, 2, 4, 2, 512, 64)
        ck = host.synth_checkpoint(cfg, 4, 32, seed=24, q4_divisor=7.0)
        steps = 40
    else:
        cfg = host.make_config(4096, 11008, 2, 32, 32, 32000, 4096)
        ck = host.synth_checkpoint(cfg, 4, 64, seed=22, q4_divisor=7.0)
        steps = 12
    print(f"engine kv8 {shape}", flush=True)
    eng = Engine(ck, max_steps=steps, kv8=True)
    assert eng.attention_splits > 0
    orc = O.Oracle(ck.cfg.as_list(), ck.weights, ck.wbits, ck.group, max_t=steps, kv8=True,
                   kv8_splits=eng.attention_splits, kv8_split_from=abi.L2Q_KV8_SPLIT_FROM)
    token = 3
    for pos in range(steps):
        lo = orc.forward(token, pos)
        lg = eng.forward(token, pos)
        np.testing.assert_array_equal(lg, lo, err_msg=f"pos {pos}")
        token = int(np.argmax(lo))
    eng.close()
    orc.close()


@pytest.mark.gpu
@pytest.mark.parametrize("shape", ["c1_q8_g32", "7b2_q4_g64", "gqa_hs64_q4_g32", "c1_q8_g32_long"])
def test_gpu_engine_kv8_prefill_follows_oracle(gpu_lib, torch_cuda, shape):
    """The batched prefill with the int8 KV cache: the qkv GEMM stages the
    rotated k, v rows, the decode step's int8 quantizer appends them, and
    each query's attention is the kernel its decode step would run (one
    workgroup per head up to L2Q_KV8_SPLIT_FROM positions, split beyond).
    The prompt's last logits and the greedy steps after it equal the
    oracle's int8-KV forward bit for bit; the long case prefills 1060
    positions in two calls, the second chunk straddling the switch."""
    from llama2q.model import Engine
    split = None
    if shape == "c1_q8_g32":
        ck = host.synth_checkpoint(host.config_15m(), 8, 32, seed=21)
        n_prompt, steps = 40, 64
    elif shape == "c1_q8_g32_long":
        cfg = host.make_config(288, 768, 2, 6, 6, 512, 2048)
        ck = host.synth_checkpoint(cfg, 8, 32, seed=25)
        n_prompt, steps, split = 1060, 1080, 1000
    elif shape == "gqa_hs64_q4_g32":
        cfg = host.make_config(256, 512, 2, 4, 2, 512, 64)
        ck = host.synth_checkpoint(cfg, 4, 32, seed=24, q4_divisor=7.0)
        n_prompt, steps = 30, 40
    else:
        cfg = host.make_config(4096, 11008, 2, 32, 32, 32000, 4096)
        ck = host.synth_checkpoint(cfg, 4, 64, seed=22, q4_divisor=7.0)
        n_prompt, steps = 9, 12
    print(f"engine kv8 prefill {shape}", flush=True)
    vocab = ck.cfg.as_list()[5]
    prompt = [int(v) for v in host.uniform_ints(n_prompt, 27, 100, 3, vocab)]
    eng = Engine(ck, max_steps=steps, kv8=True)
    orc = O.Oracle(ck.cfg.as_list(), ck.weights, ck.wbits, ck.group, max_t=steps, kv8=True,
                   kv8_splits=eng.attention_splits, kv8_split_from=abi.L2Q_KV8_SPLIT_FROM)
    for pos, tok in enumerate(prompt):
        lo = orc.forward(tok, pos)
    if split:
        eng.prefill(prompt[:split], 0, logits=False)
        lg = eng.prefill(prompt[split:], split)
    else:
        lg = eng.prefill(prompt, 0)
    np.testing.assert_array_equal(lg, lo, err_msg="last prompt position")
    token = int(np.argmax(lo))
    for pos in range(n_prompt, steps):
        lo = orc.forward(token, pos)
        lg = eng.forward(token, pos)
        np.testing.assert_array_equal(lg, lo, err_msg=f"pos {pos}")
        token = int(np.argmax(lo))
    eng.close()
    orc.close()

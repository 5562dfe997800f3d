"""Batched prefill (reference: v2-cuda/run.cu:131-162,
347-394).

l2q_gemm_q: T activation vectors against one weight matrix, group dots on
int8 MFMA, then the decode path's ordered fold: every output is compared bit
for bit with the oracle's matmul of the same vector (runq.c:142-159), at
INT8 / INT4, groups 32 / 64, with ragged rows and token counts.

l2q_engine_prefill: a prompt through every layer at once must leave the
engine exactly where token-by-token decoding leaves it: the last
position's logits equal the oracle's forward bit for bit, and greedy decode
continued from the prefilled KV cache reproduces the oracle's ids.
Prompts that cross the 128-token chunk, a prefill resumed at pos0 > 0 and
the 7B shape (INT4 g64) are covered.
"""
import numpy as np
import pytest

from llama2q import abi, host
from llama2q.model import Engine
import oracle_py as O

pytestmark = pytest.mark.gpu


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("group", [32, 64])
@pytest.mark.parametrize("rows,cols,T", [(288, 288, 1), (768, 288, 17), (4096, 4096, 128), (4096, 11008, 33),
                                         (130, 4224, 20), (3, 64, 5), (32000, 4096, 16), (4128, 4096, 100)])
def test_gemm_matches_oracle_per_token(gpu_lib, torch_cuda, bits, group, rows, cols, T):
    if cols % group:
        pytest.skip("group does not divide cols")
    t = torch_cuda
    print(f"gemm bits={bits} group={group} rows={rows} cols={cols} T={T}", flush=True)
    seed = rows + cols + T + bits + group
    w = host.gauss(rows * cols, seed, 7, 0.02).reshape(rows, cols)
    q, s = host.quantize_q8(w, group) if bits == 8 else host.quantize_q4(w, group, 7.0)
    wq = q.view(np.int8) ^ np.int8(-128) if bits == 8 else q
    xs_all, xq_all, ref = [], [], []
    for i in range(T):
        x = host.gauss(cols, seed, 100 + i, 1.0 + (i % 3))
        if i == 2:
            x[:group] = 0.0                     # an all-zero group
        xq, xs, xt = O.quantize_act(x, group)
        xq_all.append(xq)
        xs_all.append(xs)
        ref.append(O.matmul(bits, xq, xs, xt, q, s, rows, cols, group, want_dots=False)[0])
    d_w, d_s = dev(t, wq), dev(t, s)
    d_xq, d_xs = dev(t, np.stack(xq_all)), dev(t, np.stack(xs_all))
    out = t.empty(T * rows, dtype=t.float32, device="cuda")
    abi.call("l2q_gemm_q", bits, out.data_ptr(), d_xq.data_ptr(), d_xs.data_ptr(), d_w.data_ptr(), d_s.data_ptr(),
             rows, cols, group, T, t.cuda.current_stream().cuda_stream)
    t.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy().reshape(T, rows), np.stack(ref))


def prefill_then_greedy(ck, prompt, n_steps, max_steps, split=None):
    """Prefill the prompt (optionally in two calls at `split`), then greedy
    decode; the oracle runs the same positions token by token."""
    eng = Engine(ck, max_steps=max_steps)
    orc = O.Oracle(ck.cfg.as_list(), ck.weights, ck.wbits, ck.group, max_t=max_steps)
    for pos, tok in enumerate(prompt):
        lo = orc.forward(tok, pos)
    if split:
        eng.prefill(prompt[:split], 0, logits=False)
        lg = eng.prefill(prompt[split:], split)
    else:
        lg = eng.prefill(prompt, 0)
    np.testing.assert_array_equal(lg, lo, err_msg="logits of the last prompt position")
    token, pos = int(np.argmax(lo)), len(prompt)
    for _ in range(n_steps):
        lo = orc.forward(token, pos)
        lg = eng.forward(token, pos)
        np.testing.assert_array_equal(lg, lo, err_msg=f"decode after prefill, pos {pos}")
        token, pos = int(np.argmax(lo)), pos + 1
    eng.close()
    orc.close()


@pytest.fixture(scope="module")
def c1_q8():
    return host.synth_checkpoint(host.config_15m(), 8, 32, seed=4321)


@pytest.mark.parametrize("n_prompt,split", [(1, None), (16, None), (16, 5), (200, None)])
def test_engine_prefill_c1_q8(gpu_lib, c1_q8, n_prompt, split):
    print(f"prefill c1 q8 n={n_prompt} split={split}", flush=True)
    prompt = [int(v) for v in host.uniform_ints(n_prompt, 77, 100, 3, 32000)]
    prefill_then_greedy(c1_q8, prompt, 12, 256, split)


@pytest.mark.parametrize("max_steps", [61, 150])
def test_engine_prefill_cache_length_not_multiple_of_4(gpu_lib, c1_q8, max_steps):
    """A KV cache of 61 / 150 positions: the batched attention's score rows
    are padded to a multiple of 4 internally (its float4 reads), so such
    engines run the same batched kernels and stay bit-exact."""
    print(f"prefill c1 q8 max_steps={max_steps}", flush=True)
    prompt = [int(v) for v in host.uniform_ints(min(50, max_steps - 8), 78, 100, 3, 32000)]
    prefill_then_greedy(c1_q8, prompt, 6, max_steps)


def test_engine_prefill_c1_q4_g32(gpu_lib):
    ck = host.synth_checkpoint(host.config_15m(), 4, 32, seed=99, q4_divisor=8.0)
    prompt = [int(v) for v in host.uniform_ints(40, 5, 100, 3, 32000)]
    prefill_then_greedy(ck, prompt, 8, 64)


def test_engine_prefill_7b_shape_int4_g64(gpu_lib):
    cfg = host.make_config(4096, 11008, 2, 32, 32, 32000, 4096)
    ck = host.synth_checkpoint(cfg, 4, 64, seed=23, q4_divisor=7.0)
    prompt = [int(v) for v in host.uniform_ints(40, 6, 100, 3, 32000)]
    prefill_then_greedy(ck, prompt, 4, 64)


@pytest.mark.parametrize("bits,group", [(4, 64), (8, 32), (8, 64), (4, 32)])
@pytest.mark.parametrize("n_prompt,split", [(300, None), (200, 150)])
def test_engine_prefill_fused_attention_chunks(gpu_lib, bits, group, n_prompt, split):
    """Head size 128 (the fused softmax + p*V + quantize attention): a
    300-position prompt prefills in chunks at positions 0, 128 (contexts of
    up to 256: the fused kernel) and 256 (the three-kernel path); a second
    call at pos0 = 150 mixes both; bit-exact against the oracle.  The four
    bit widths x group sizes also cover every form of the w1|w3 GEMM's
    SwiGLU + Q8 stores."""
    print(f"prefill hs128 bits={bits} group={group} n={n_prompt} split={split}", flush=True)
    cfg = host.make_config(512, 1024, 2, 4, 4, 32000, 512)
    ck = host.synth_checkpoint(cfg, bits, group, seed=31 + bits, q4_divisor=7.0)
    prompt = [int(v) for v in host.uniform_ints(n_prompt, 8, 100, 3, 32000)]
    prefill_then_greedy(ck, prompt, 4, 512, split)


def test_engine_prefill_rejects_bad_positions(gpu_lib, c1_q8):
    eng = Engine(c1_q8, max_steps=32)
    toks = np.arange(3, 13, dtype=np.int32)
    for pos0, n in ((30, 5), (-1, 2)):
        rc = abi.lib().l2q_engine_prefill(eng._h, toks.ctypes.data, n, pos0, None)
        assert rc in (abi.L2Q_ERR_STATE, abi.L2Q_ERR_ARG)
    bad = np.array([5, 40000], dtype=np.int32)
    assert abi.lib().l2q_engine_prefill(eng._h, bad.ctypes.data, 2, 0, None) == abi.L2Q_ERR_ARG
    eng.close()


@pytest.mark.parametrize("shape", ["15m", "7b"])
def test_engine_prefill_denormal_embedding(gpu_lib, shape):
    """The embedding table scaled by 1e-42: the batched prefill's RMSNorm,
    SwiGLU and quantize kernels meet denormal residual streams and group
    scales where the reference's clamp to +-127 binds; the last prompt
    position's logits and the decode after it equal the reference's."""
    if shape == "7b":
        cfg = host.make_config(4096, 11008, 2, 32, 32, 32000, 4096)
        ck = host.synth_checkpoint(cfg, 4, 64, seed=29, q4_divisor=7.0)
    else:
        cfg = host.config_15m()
        ck = host.synth_checkpoint(cfg, 4, 32, seed=31, q4_divisor=8.0)
    off = ck.layout().emb
    emb = ck.weights[off:off + cfg.vocab_size * cfg.dim * 4].view(np.float32)
    emb *= np.float32(1e-42)
    prompt = [int(v) for v in host.uniform_ints(24, 8, 100, 3, 32000)]
    prefill_then_greedy(ck, prompt, 4, 64)


@pytest.mark.parametrize("bits", [8, 4])
def test_engine_prefill_gqa_hs64(gpu_lib, bits):
    """Batched prefill of a grouped-query model (4 heads over 2 kv heads,
    heads of 64, groups of 32), in two calls: logits and the decode after it
    equal the reference's."""
    cfg = host.make_config(256, 512, 2, 4, 2, 512, 64)
    kw = {"q4_divisor": 7.0} if bits == 4 else {}
    ck = host.synth_checkpoint(cfg, bits, 32, seed=15 + bits, **kw)
    prompt = [int(v) for v in host.uniform_ints(30, 9, 100, 3, 512)]
    prefill_then_greedy(ck, prompt, 6, 64, split=11)

"""l2q_attention_split_noalloc (the allocation-free form of
l2q_attention_split, its partials in a static per-GPU scratch array) against
l2q_attention_split, both through the C ABI: identical outputs on two calls
in a row, the second smaller than the first, and a clear error when the
partials would not fit the static array."""
import pytest

from llama2q import abi

pytestmark = pytest.mark.gpu


def _attend(torch, name, q, k, v, pos, heads, kv_heads, hs, max_t):
    out = torch.full((heads * hs,), float("nan"), device="cuda")
    abi.call(name, q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), pos, heads, kv_heads, hs, max_t,
             torch.cuda.current_stream().cuda_stream)
    return out


def test_noalloc_split_equals_split_twice(gpu_lib, torch_cuda):
    torch = torch_cuda
    g = torch.Generator(device="cuda")
    g.manual_seed(11)
    # (heads, kv heads, head size, cache positions, pos): config 4 at a long
    # context, then a smaller grouped-query call reusing the same scratch
    for heads, kv_heads, hs, max_t, pos in ((32, 32, 128, 4096, 3000), (8, 2, 64, 512, 200)):
        q = torch.randn(heads * hs, device="cuda", generator=g)
        k = torch.randn(kv_heads * max_t * hs, device="cuda", generator=g)
        v = torch.randn(kv_heads * max_t * hs, device="cuda", generator=g)
        want = _attend(torch, "l2q_attention_split", q, k, v, pos, heads, kv_heads, hs, max_t)
        got = _attend(torch, "l2q_attention_split_noalloc", q, k, v, pos, heads, kv_heads, hs, max_t)
        torch.cuda.synchronize()
        assert torch.isfinite(want).all()
        assert torch.equal(got, want), f"heads={heads} hs={hs} pos={pos}"


def test_noalloc_split_rejects_partials_beyond_the_static_scratch(gpu_lib, torch_cuda):
    torch = torch_cuda
    x = torch.zeros(64, device="cuda")
    # 64 heads x 512 splits x (256 + 2) floats > 2^20: refused before any launch
    with pytest.raises(abi.L2QError, match="static scratch"):
        abi.call("l2q_attention_split_noalloc", x.data_ptr(), x.data_ptr(), x.data_ptr(), x.data_ptr(), 65535, 64, 64,
                 256, 65536, torch.cuda.current_stream().cuda_stream)

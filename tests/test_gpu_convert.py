"""The library's conversion and zero-fill entry points (fc_convert,
fc_fill_zero), which a Julia binding uses for attention_inputs
(ext/FemtoChatCUDAExt.jl:229-230) and zeroed gradients instead of device
broadcasts: float32 -> bfloat16 is bit-exact against torch's conversion
(round to nearest even, ties included), bfloat16 -> float32 is exact, on
vector and scalar paths (sizes that are not multiples of 8, pointers that are
not 16-byte aligned); the fill writes exactly the requested bytes.
"""
import numpy as np
import pytest
import torch

from femtochat_amd import MFMAExact, MFMAFast, attention_inputs, convert_, fill_zero_

pytestmark = pytest.mark.gpu


def _specials():
    # ties between two bf16 values (both parities), the largest finite values,
    # float32 and bfloat16 subnormals, zeros, infinities
    vals = [1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, -(1.0 + 2.0 ** -8), 3.3895313892515355e38, -3.3895313892515355e38,
            2.0 ** -130, -(2.0 ** -133), 1e-40, 2.0 ** -126, 0.0, -0.0, float("inf"), float("-inf")]
    return torch.tensor(vals, dtype=torch.float32)


def _f32_cases(n, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(n, generator=g) * torch.pow(10.0, torch.randint(-30, 31, (n,), generator=g).float())
    x[: min(n, 13)] = _specials()[: min(n, 13)]
    return x


@pytest.mark.parametrize("n", [8, 13, 1000, 4096 * 37 + 5])
@pytest.mark.parametrize("offset", [0, 1])
def test_f32_to_bf16_is_bit_exact(gpu, n, offset):
    x = _f32_cases(n + offset, seed=n)
    src = x.to(gpu)[offset:]  # offset 1: a 4-byte, not 16-byte, aligned source
    dst_buf = torch.empty(n + offset, dtype=torch.bfloat16, device=gpu)
    dst = dst_buf[offset:]
    convert_(dst, src)
    torch.cuda.synchronize()
    ref = src.cpu().to(torch.bfloat16)
    assert torch.equal(dst.cpu().view(torch.int16), ref.view(torch.int16))


def test_nan_stays_nan(gpu):
    x = torch.tensor([float("nan"), 1.0, -float("nan"), 2.0] * 4, device=gpu)
    y = torch.empty(16, dtype=torch.bfloat16, device=gpu)
    convert_(y, x)
    back = torch.empty(16, dtype=torch.float32, device=gpu)
    convert_(back, y)
    torch.cuda.synchronize()
    assert torch.equal(torch.isnan(y.cpu()), torch.isnan(x.cpu()))
    assert torch.equal(torch.isnan(back.cpu()), torch.isnan(x.cpu()))


@pytest.mark.parametrize("n", [8, 29, 100003])
@pytest.mark.parametrize("offset", [0, 3])
def test_bf16_to_f32_is_exact(gpu, n, offset):
    bits = torch.randint(-32768, 32767, (n + offset,), generator=torch.Generator().manual_seed(n), dtype=torch.int16)
    bits[(bits & 0x7F80) == 0x7F80] = 0x3F80  # no NaN/Inf patterns here (NaN is tested above)
    src = bits.view(torch.bfloat16).to(gpu)[offset:]
    dst = torch.empty(n, dtype=torch.float32, device=gpu)
    convert_(dst, src)
    torch.cuda.synchronize()
    assert torch.equal(dst.cpu(), src.cpu().to(torch.float32))


def test_same_dtype_copies(gpu):
    x = torch.randn(1001, device=gpu)
    y = torch.empty_like(x)
    convert_(y, x)
    torch.cuda.synchronize()
    assert torch.equal(x, y)


@pytest.mark.parametrize("nbytes,offset", [(1, 0), (15, 3), (16, 0), (4096, 8), (1_000_003, 5)])
def test_fill_zero_writes_exactly_the_range(gpu, nbytes, offset):
    buf = torch.full((nbytes + offset + 32,), 0xAB, dtype=torch.uint8, device=gpu)
    fill_zero_(buf[offset:offset + nbytes])
    torch.cuda.synchronize()
    h = buf.cpu().numpy()
    assert np.all(h[offset:offset + nbytes] == 0)
    assert np.all(h[:offset] == 0xAB) and np.all(h[offset + nbytes:] == 0xAB)


def test_attention_inputs_convert_through_the_library(gpu):
    g = torch.Generator(device=gpu).manual_seed(3)
    Q, K, V = (torch.randn(2, 33, h, 64, device=gpu, generator=g) for h in (4, 2, 2))
    q, k, v = attention_inputs(MFMAFast(), Q, K, V)
    assert q.dtype == k.dtype == v.dtype == torch.bfloat16
    for a, b in zip((q, k, v), (Q, K, V)):
        assert torch.equal(a.view(torch.int16), b.to(torch.bfloat16).view(torch.int16))
    q2, k2, v2 = attention_inputs(MFMAExact(), q, k, v)
    assert q2.dtype == torch.float32 and torch.equal(q2, q.float())

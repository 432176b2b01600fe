"""Rows scaled into float16 by a power of two each (strata_rows_to_f16) and products scaled back
(strata_rows_from_f32): the bits of a torch restatement of the same arithmetic. rows_to_f16 puts each row's largest
magnitude into [2^14, 2^15) by e = floor(log2 max) - 14 (0 for a row of zeros, or one holding an infinity or a NaN)
and rounds x / 2^e to float16; rows_from_f32 rounds c * 2^e once to the output type. Row lengths that take the
single-read form (multiples of 8 up to 8192) and ones that do not, a zero row, a row holding an infinity and rows
spanning many binades."""

import numpy as np
import pytest
import torch

from strata_mlx_amd import blocks as B

pytestmark = pytest.mark.gpu


def exponents(x: torch.Tensor) -> torch.Tensor:
    m = x.float().abs().amax(dim=1)
    _, ex = torch.frexp(m)
    return torch.where((m > 0) & torch.isfinite(m), ex - 15, torch.zeros_like(ex))


def rows(cols: int, dtype, gpu) -> torch.Tensor:
    rng = np.random.default_rng(cols)
    x = rng.standard_normal((6, cols)) * np.exp2(rng.integers(-20, 20, (6, 1)))
    x[1] = 0.0                                      # a row of zeros
    x[2, 3] = np.inf                                # a row holding an infinity
    x[3] *= np.exp2(rng.integers(-12, 12, cols))    # values over many binades
    x[4, :] = 70000.0 * np.sign(x[4])               # past float16's range, before scaling
    return torch.from_numpy(x.astype(np.float32)).to(dtype).to(gpu)


@pytest.mark.parametrize("cols", [1536, 4096, 8192, 1000, 8200])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_rows_to_f16_is_the_scaled_rounding(gpu, cols, dtype):
    x = rows(cols, dtype, gpu)
    got, row_max = B.rows_to_f16(x)
    e = exponents(x).cpu().numpy()
    # numpy's float32 -> float16 conversion rounds to nearest even also in the subnormal range, ties included
    with np.errstate(over="ignore"):  # values past float16's range, as in the kernel, become infinities
        want = (x.float().cpu().numpy() * np.exp2(-e[:, None]).astype(np.float32)).astype(np.float16)
    assert np.array_equal(got.cpu().numpy().view(np.uint16), want.view(np.uint16))
    m = x.float().abs().amax(dim=1)
    finite = torch.isfinite(m)
    assert torch.equal(row_max.view(torch.float32)[finite], m[finite])


@pytest.mark.parametrize("cols", [12288, 1537])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_rows_from_f32_rounds_once(gpu, cols, dtype):
    x = rows(4096, torch.bfloat16, gpu)
    _, row_max = B.rows_to_f16(x)
    c = torch.from_numpy(np.random.default_rng(5).standard_normal((6, cols)).astype(np.float32) * 3e4).to(gpu)
    got = B.rows_from_f32(c, row_max, dtype)
    scaled = c.cpu().numpy() * np.exp2(exponents(x).cpu().numpy()[:, None]).astype(np.float32)  # exact
    if dtype == torch.bfloat16:  # round to nearest even at bit 16 of the float32 pattern
        u = scaled.view(np.uint32).astype(np.uint64)
        want = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
        assert np.array_equal(got.view(torch.int16).cpu().numpy().view(np.uint16), want)
    elif dtype == torch.float16:
        with np.errstate(over="ignore"):
            want = scaled.astype(np.float16)
        assert np.array_equal(got.cpu().numpy().view(np.uint16), want.view(np.uint16))
    else:
        assert np.array_equal(got.cpu().numpy(), scaled)

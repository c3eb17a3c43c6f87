"""The prompt pass's elementwise kernels (egpt_silu_mul, egpt_add_rmsnorm, egpt_rmsnorm) in their two forms.

Rows of whole 16-byte groups take the vector kernels (16-byte accesses, 8 elements per
thread); other rows the scalar ones. Per element both forms compute transformers' bf16
Qwen3 roundings (models/qwen3/modeling_qwen3.py: SwiGLU bf16(bf16(silu(g)) * u) :49-62,
residual bf16(x + a) and RMSNorm bf16(w * bf16(x * rsqrt(mean x^2 + eps))) :30-46,
:285-322). SwiGLU is therefore bit-identical between the forms; the residual update
too. The norm's mean of squares is an fp32 sum in another order, and rsqrtf is not
correctly rounded: where x * inv sits at a bf16 rounding boundary its rounding can flip,
which the weight's product and the last rounding turn into up to two and a half ulps of
the output. So the forms agree bit for bit on 99% of the elements and to two ulps on
all, and both match an fp64 restatement of the formula to three.
"""

import numpy as np
import pytest
import torch

from efficientgpt_amd import _lib

pytestmark = pytest.mark.gpu


def _ulp(v):
    a = np.abs(np.asarray(v, np.float64))
    a = np.where(a == 0, 1e-38, a)
    return 2.0 ** (np.floor(np.log2(a)) - 7)


@pytest.mark.parametrize('rows,inter', [(8192, 12288), (37, 6144), (5, 40)])
def test_silu_mul_vector_and_scalar_forms_agree(rows, inter):
    lib = _lib.lib()
    g = torch.Generator().manual_seed(rows + inter)
    gu = (torch.randn(rows, 2 * inter, generator=g) * 3).to(torch.bfloat16)
    dev = gu.cuda()
    out_v = torch.empty(rows, inter, device='cuda', dtype=torch.bfloat16)
    assert lib.egpt_silu_mul(dev.data_ptr(), 2 * inter, inter, out_v.data_ptr(), inter, rows, _lib.stream_ptr()) == 0
    # the same rows one element off 16-byte alignment: the scalar kernel
    wide = torch.zeros(rows, 2 * inter + 1, dtype=torch.bfloat16, device='cuda')
    wide[:, 1:] = dev
    out_s = torch.zeros(rows, inter + 1, device='cuda', dtype=torch.bfloat16)
    assert lib.egpt_silu_mul(wide[:, 1:].data_ptr(), 2 * inter + 1, inter, out_s[:, 1:].data_ptr(), inter + 1, rows,
                             _lib.stream_ptr()) == 0
    torch.cuda.synchronize()
    assert torch.equal(out_v, out_s[:, 1:])
    gf, uf = gu[:, :inter].float(), gu[:, inter:].float()
    want = ((gf / (1 + torch.exp(-gf))).to(torch.bfloat16).float() * uf).to(torch.bfloat16)
    diff = np.abs(out_v.float().cpu().numpy().astype(np.float64) - want.float().numpy())
    assert np.all(diff <= _ulp(want.float().numpy())), float(diff.max())
    assert np.mean(diff == 0) >= 0.999


@pytest.mark.parametrize('rows,n', [(8192, 4096), (64, 2048), (3, 1000), (4, 100)])
def test_add_rmsnorm_vector_and_scalar_forms_agree(rows, n):
    lib = _lib.lib()
    g = torch.Generator().manual_seed(rows * 3 + n)
    x = torch.randn(rows, n, generator=g).to(torch.bfloat16)
    a = (torch.randn(rows, n, generator=g) * 2).to(torch.bfloat16)
    w = (1 + 0.2 * torch.randn(n, generator=g)).to(torch.bfloat16)
    st = _lib.stream_ptr()
    xv, av, wv = x.cuda(), a.cuda(), w.cuda()
    yv = torch.empty(rows, n, device='cuda', dtype=torch.bfloat16)
    assert lib.egpt_add_rmsnorm(xv.data_ptr(), n, av.data_ptr(), n, wv.data_ptr(), yv.data_ptr(), n, rows, n, 1e-6,
                                st) == 0
    # rows one element off alignment: the scalar kernel
    xs = torch.zeros(rows, n + 1, dtype=torch.bfloat16, device='cuda')
    xs[:, 1:] = x.cuda()
    ys = torch.zeros(rows, n + 1, dtype=torch.bfloat16, device='cuda')
    assert lib.egpt_add_rmsnorm(xs[:, 1:].data_ptr(), n + 1, av.data_ptr(), n, wv.data_ptr(), ys[:, 1:].data_ptr(),
                                n + 1, rows, n, 1e-6, st) == 0
    # the norm alone (egpt_rmsnorm) over the updated rows
    yn = torch.empty(rows, n, device='cuda', dtype=torch.bfloat16)
    assert lib.egpt_rmsnorm(xv.data_ptr(), n, wv.data_ptr(), yn.data_ptr(), n, rows, n, 1e-6, st) == 0
    torch.cuda.synchronize()
    assert torch.equal(xv, xs[:, 1:])  # the residual update: bf16(x + a), bit-identical
    r = (x.float() + a.float()).to(torch.bfloat16)
    assert torch.equal(xv.cpu(), r)
    rf = r.double().numpy()
    inv = 1.0 / np.sqrt((rf * rf).mean(axis=1, keepdims=True) + 1e-6)
    normed = torch.from_numpy(rf * inv).to(torch.bfloat16).double().numpy()
    want = torch.from_numpy(w.double().numpy()[None, :] * normed).to(torch.bfloat16).double().numpy()
    for y in (yv, ys[:, 1:], yn):
        got = y.double().cpu().numpy()
        assert np.all(np.abs(got - want) <= 3 * _ulp(want)), float((np.abs(got - want) / _ulp(want)).max())
    dvs = np.abs(yv.double().cpu().numpy() - ys[:, 1:].double().cpu().numpy())
    assert np.all(dvs <= 2 * _ulp(want)) and np.mean(dvs == 0) >= 0.99
    assert torch.equal(yv, yn)  # the same vector kernel over the same rows

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

import ctypes

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


@pytest.mark.parametrize('d,hq,hkv,rows', [(128, 32, 8, 4096), (128, 16, 8, 100), (64, 6, 6, 33), (32, 4, 2, 17)])
def test_qk_norm_rope_vector_and_scalar_forms_agree(d, hq, hkv, rows):
    """egpt_qk_norm_rope over a prompt block: query heads normalised and rotated into q_out, key heads into the key
    cache at each row's position, value heads copied into the value cache. The vector form (16-byte rows) against
    the wavefront-per-head form (rows one element off alignment): value copies bit-identical, normalised heads to
    two bf16 ulps of the larger RoPE term (the head's mean of squares in another fp32 order) and 99% bit-identical;
    both within three such ulps of an fp64 restatement of transformers' q/k norm and RoPE (modeling_qwen3.py:
    139-166, 237-256)."""
    lib = _lib.lib()
    g = torch.Generator().manual_seed(d + hq + rows)
    cap, pos0 = rows + 40, 25
    n = (hq + 2 * hkv) * d
    qkv = torch.randn(rows, n, generator=g).to(torch.bfloat16)
    qn = (1 + 0.2 * torch.randn(d, generator=g)).to(torch.bfloat16)
    kn = (1 + 0.2 * torch.randn(d, generator=g)).to(torch.bfloat16)
    inv_freq = 1.0 / (1e6 ** (torch.arange(0, d, 2, dtype=torch.float) / d))
    ang = torch.arange(cap, dtype=torch.float)[:, None] * inv_freq[None, :]
    emb = torch.cat([ang, ang], 1)
    cos, sin = emb.cos().to(torch.bfloat16), emb.sin().to(torch.bfloat16)
    positions = torch.arange(pos0, pos0 + rows, dtype=torch.long)
    st = _lib.stream_ptr()

    def run(offset):
        src = torch.zeros(rows, n + offset, dtype=torch.bfloat16, device='cuda')
        src[:, offset:] = qkv.cuda()
        q = torch.zeros(rows, hq * d + offset, dtype=torch.bfloat16, device='cuda')
        kc = torch.zeros(hkv, cap, d, dtype=torch.bfloat16, device='cuda')
        vc = torch.zeros_like(kc)
        assert lib.egpt_qk_norm_rope(src[:, offset:].data_ptr(), n + offset, positions.cuda().data_ptr(),
                                     qn.cuda().data_ptr(), kn.cuda().data_ptr(), cos.cuda().data_ptr(),
                                     sin.cuda().data_ptr(), q[:, offset:].data_ptr(), hq * d + offset, kc.data_ptr(),
                                     vc.data_ptr(), kc.stride(0), kc.stride(1), rows, hq, hkv, d, cap, 1e-6, st) == 0
        torch.cuda.synchronize()
        return q[:, offset:].cpu(), kc.cpu(), vc.cpu()

    qv, kv, vv = run(0)
    qs, ks, vs = run(1)
    assert torch.equal(vv, vs)
    assert torch.equal(vv[:, pos0:pos0 + rows], qkv[:, (hq + hkv) * d:].view(rows, hkv, d).transpose(0, 1))

    def truth(x, w):  # x [rows, heads, d] bf16 -> (the roundings in fp64, the larger of the two RoPE terms)
        xf = x.double()
        normed = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)).to(torch.bfloat16).double()
        normed = (w.double() * normed).to(torch.bfloat16).double()
        rot = torch.cat([-normed[..., d // 2:], normed[..., :d // 2]], -1)
        c, s = cos[positions].double()[:, None], sin[positions].double()[:, None]
        a, b = (normed * c).to(torch.bfloat16).double(), (rot * s).to(torch.bfloat16).double()
        return (a + b).to(torch.bfloat16), torch.maximum(a.abs(), b.abs())

    want_q, mag_q = truth(qkv[:, :hq * d].view(rows, hq, d), qn)
    want_k, mag_k = truth(qkv[:, hq * d:(hq + hkv) * d].view(rows, hkv, d), kn)
    cases = ((qv, qs, want_q.view(rows, hq * d), mag_q.view(rows, hq * d)),
             (kv[:, pos0:pos0 + rows], ks[:, pos0:pos0 + rows], want_k.transpose(0, 1), mag_k.transpose(0, 1)))
    for got, other, want, mag in cases:
        # a flipped rounding of a normalised element moves each RoPE term by up to an ulp of that term: near a
        # cancelling sum that is many ulps of the result, so the bound is in ulps of the larger term
        w64, unit = want.double().numpy(), _ulp(np.maximum(np.abs(want.double().numpy()), mag.numpy()))
        for y in (got, other):
            dd = np.abs(y.double().numpy() - w64)
            assert np.all(dd <= 3 * unit), float((dd / unit).max())
        dvs = np.abs(got.double().numpy() - other.double().numpy())
        assert np.all(dvs <= 2 * unit) and np.mean(dvs == 0) >= 0.99


@pytest.mark.parametrize('d,hq,hkv,rows,k', [(128, 16, 8, 128, 2048), (128, 32, 8, 40, 4096), (128, 8, 4, 200, 2048),
                                             (64, 4, 2, 64, 1024), (32, 4, 2, 17, 2048)])
def test_gemm_qk_norm_rope_matches_the_two_calls_bit_for_bit(d, hq, hkv, rows, k):
    """egpt_int8_gemm_qk_norm_rope (the split-K QKV product whose reduce also runs q/k norm, RoPE and the cache
    writes) against egpt_int8_gemm_ws into a qkv buffer followed by egpt_qk_norm_rope: rotated queries, key and
    value caches the same bits; the rows it does not write stay as they were. A shape whose product does not split
    K, and a short workspace, are refused before any launch."""
    lib = _lib.lib()
    g = torch.Generator().manual_seed(d + hq + rows + k)
    n = (hq + 2 * hkv) * d
    cap, pos0 = rows + 40, 25
    x = torch.randn(rows, k, generator=g).to(torch.bfloat16).cuda()
    w = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8).cuda()
    s = (torch.rand(n, generator=g) * 0.02 + 1e-3).cuda()
    qn = (1 + 0.2 * torch.randn(d, generator=g)).to(torch.bfloat16).cuda()
    kn = (1 + 0.2 * torch.randn(d, generator=g)).to(torch.bfloat16).cuda()
    inv_freq = 1.0 / (1e6 ** (torch.arange(0, d, 2, dtype=torch.float) / d))
    ang = torch.arange(cap, dtype=torch.float)[:, None] * inv_freq[None, :]
    emb = torch.cat([ang, ang], 1)
    cos, sin = emb.cos().to(torch.bfloat16).cuda(), emb.sin().to(torch.bfloat16).cuda()
    positions = torch.arange(pos0, pos0 + rows, dtype=torch.long).cuda()
    need = ctypes.c_size_t()
    assert lib.egpt_int8_gemm_workspace(rows, n, k, ctypes.byref(need)) == 0
    assert need.value > 0, 'the case must split K'
    ws = torch.empty(need.value, dtype=torch.uint8, device='cuda')
    st = _lib.stream_ptr()
    out = []
    for fused in (True, False):
        q = torch.full((rows, hq * d), float('nan'), dtype=torch.bfloat16, device='cuda')
        kc = torch.full((hkv, cap, d), 7.0, dtype=torch.bfloat16, device='cuda')
        vc = torch.full_like(kc, -7.0)
        if fused:
            assert lib.egpt_int8_gemm_qk_norm_rope(
                x.data_ptr(), k, w.data_ptr(), k, s.data_ptr(), positions.data_ptr(), qn.data_ptr(), kn.data_ptr(),
                cos.data_ptr(), sin.data_ptr(), q.data_ptr(), hq * d, kc.data_ptr(), vc.data_ptr(), kc.stride(0),
                kc.stride(1), rows, hq, hkv, d, k, cap, 1e-6, ws.data_ptr(), ws.numel(), st) == 0
        else:
            qkv = torch.empty(rows, n, dtype=torch.bfloat16, device='cuda')
            assert lib.egpt_int8_gemm_ws(x.data_ptr(), k, w.data_ptr(), k, s.data_ptr(), qkv.data_ptr(), n, rows, n,
                                         k, ws.data_ptr(), ws.numel(), st) == 0
            assert lib.egpt_qk_norm_rope(qkv.data_ptr(), n, positions.data_ptr(), qn.data_ptr(), kn.data_ptr(),
                                         cos.data_ptr(), sin.data_ptr(), q.data_ptr(), hq * d, kc.data_ptr(),
                                         vc.data_ptr(), kc.stride(0), kc.stride(1), rows, hq, hkv, d, cap, 1e-6,
                                         st) == 0
        torch.cuda.synchronize()
        out.append((q.cpu(), kc.cpu(), vc.cpu()))
    (qa, ka, va), (qb, kb, vb) = out
    assert torch.equal(qa, qb) and not bool(torch.isnan(qa.float()).any())
    assert torch.equal(ka, kb) and torch.equal(va, vb)
    assert bool((ka[:, :pos0] == 7).all()) and bool((va[:, pos0 + rows:] == -7).all())
    args = (positions.data_ptr(), qn.data_ptr(), kn.data_ptr(), cos.data_ptr(), sin.data_ptr(), q.data_ptr(), hq * d,
            kc.data_ptr(), vc.data_ptr(), kc.stride(0), kc.stride(1))
    assert lib.egpt_int8_gemm_qk_norm_rope(x.data_ptr(), k, w.data_ptr(), k, s.data_ptr(), *args, rows, hq, hkv, d,
                                           k, cap, 1e-6, ws.data_ptr(), need.value - 4,
                                           st) == _lib.EGPT_ERR_WORKSPACE
    # 1024 rows: the product's tiles fill the chip, K is not split
    assert lib.egpt_int8_gemm_qk_norm_rope(x.data_ptr(), k, w.data_ptr(), k, s.data_ptr(), *args, 1024, hq, hkv, d,
                                           k, cap, 1e-6, ws.data_ptr(), ws.numel(),
                                           st) == _lib.EGPT_ERR_UNSUPPORTED

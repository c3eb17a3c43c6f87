"""HIP int8 GEMV vs the CPU oracle: the reference's tolerance rules plus bf16-ulp agreement with the oracle formula.

Mirrors research/realmodel/test_int8_linear.py (shapes, split-K configs, row guard,
model surgery, graph capture) and the KernelAgent int8_gemv edge cases
(research/kernelagent/tasks.py:132-158: x * 30, weights at +-127).
"""

import numpy as np
import pytest
import torch

from oracle import int8 as oint8

pytestmark = pytest.mark.gpu

REFERENCE_SHAPES = [(1, 2048, 6144), (4, 6144, 2048), (16, 2048, 1024), (3, 100, 70), (17, 2048, 512), (64, 512, 256)]
QWEN3_SHAPES = [(1, 2048, 4096), (1, 2048, 2048), (1, 2048, 12288), (1, 6144, 2048), (2, 2048, 4096),
                (8, 2048, 2048), (1, 4096, 4096), (1, 12288, 4096), (1, 1024, 48), (1, 3072, 256)]


def make_case(m, k, n, seed=0, edge=None):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=g)
    if edge == 'large':
        x = x * 30.0
    q = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
    if edge == 'extreme_w':
        q = torch.where(q >= 0, torch.tensor(127, dtype=torch.int8), torch.tensor(-127, dtype=torch.int8))
    s = torch.rand(n, generator=g) * 0.02 + 1e-3
    return x.to(torch.bfloat16), q, s


def bf16_ulp(y):
    a = np.abs(np.asarray(y, np.float64))
    a = np.where(a == 0, 1e-38, a)
    return 2.0 ** (np.floor(np.log2(a)) - 7)


def check_against_oracle(y, x, q, s, min_exact=0.99):
    """Reference tolerance vs fp64 truth, and within one bf16 ulp of the oracle's formula for the row count.

    Past 16 rows the op takes the prefill GEMM (the reference's formula, two bf16
    roundings), and up to 16 rows the GEMV kernels (one rounding). Their fp32 sums
    over K run in the kernels' orders (lane chunks and DPP reductions, or the MFMA's);
    the oracle sums exactly. An
    fp32 sum of K terms is off by about sqrt(K) 2^-24 sum|x q| (a random-walk bound),
    which near a cancelling zero is many ulps of a tiny output. So there each element
    may differ by that sum error times the scale plus one ulp per rounding (three for
    the two-rounding prefill form); 90 % (prefill) or 99 % must be bit-exact. torch's own
    bf16 GEMM of the same formula needs the allowance too (up to 99 ulps at outputs near
    1e-6 on these shapes).
    """
    prefill = x.shape[0] > oint8.MAX_DECODE_ROWS
    min_exact = 0.9 if prefill else min_exact
    yn = y.float().cpu().numpy()
    xn, qn, sn = x.float().numpy(), q.numpy(), s.numpy()
    err = oint8.max_err(yn, xn, qn, sn)
    assert err <= oint8.tolerance_vs_naive(xn, qn, sn), err
    want = oint8.linear(xn, qn, sn)
    diff = np.abs(yn.astype(np.float64) - want)
    sum_abs = (np.abs(xn).astype(np.float64) @ np.abs(qn).astype(np.float64).T) * sn[None, :]
    sum_err = 2.0 ** -24 * np.sqrt(xn.shape[1]) * sum_abs
    if prefill:
        bound = 3.0 * bf16_ulp(want) + sum_err
    else:  # one rounding of an fp32 sum taken in the kernel's order
        bound = bf16_ulp(want) + sum_err
    assert np.all(diff <= bound), float((diff - bound).max())
    assert np.mean(diff == 0) >= min_exact, float(np.mean(diff == 0))
    rel = np.abs(yn - oint8.linear_truth(xn, qn, sn)).max() / max(np.abs(oint8.linear_truth(xn, qn, sn)).max(), 1e-30)
    assert rel <= 2e-2


@pytest.mark.parametrize('m,k,n', REFERENCE_SHAPES + QWEN3_SHAPES)
def test_gemv_matches_oracle(m, k, n):
    from efficientgpt_amd.int8_linear import int8_linear
    x, q, s = make_case(m, k, n, seed=m * 7 + n)
    y = int8_linear(x.cuda(), q.cuda(), s.cuda())
    assert y.shape == (m, n) and y.dtype == torch.bfloat16
    check_against_oracle(y, x, q, s)


@pytest.mark.parametrize('edge', ['large', 'extreme_w'])
def test_gemv_edges(edge):
    from efficientgpt_amd.int8_linear import int8_linear
    for m, k, n in [(1, 2048, 6144), (4, 2048, 1024)]:
        x, q, s = make_case(m, k, n, seed=5, edge=edge)
        check_against_oracle(int8_linear(x.cuda(), q.cuda(), s.cuda()), x, q, s)


def test_lm_head_shape():
    from efficientgpt_amd.int8_linear import int8_linear
    x, q, s = make_case(1, 2048, 151936, seed=11)
    check_against_oracle(int8_linear(x.cuda(), q.cuda(), s.cuda()), x, q, s)


@pytest.mark.parametrize('m', [2, 4, 8])
def test_lm_head_small_batch(m):
    """The Qwen3 lm_head (151936 x 2048) at 2, 4 and 8 rows: the few-rows vector kernel at 2 rows, the LDS-staged
    MFMA form (outputs past 8192 features, K 2048) at 4 and 8."""
    from efficientgpt_amd.int8_linear import int8_linear
    x, q, s = make_case(m, 2048, 151936, seed=11 + m)
    check_against_oracle(int8_linear(x.cuda(), q.cuda(), s.cuda()), x, q, s)


@pytest.mark.parametrize('m,k,n,config', [(2, 2048, 1024, ('dot16_splitk', 64, 128, 4, 4)),
                                          (1, 6144, 2048, ('dot16_splitk', 32, 256, 8, 4)),
                                          (3, 100, 70, ('dot16_splitk', 32, 64, 3, 4))])
def test_splitk_configs(m, k, n, config):
    from efficientgpt_amd import int8_linear as mod
    x, q, s = make_case(m, k, n, seed=3)
    mod.CONFIGS[(k, n)] = config
    try:
        y = mod.int8_linear(x.cuda(), q.cuda(), s.cuda())
    finally:
        mod.CONFIGS.pop((k, n), None)
    check_against_oracle(y, x, q, s)


def test_unaligned_and_strided_operands_take_the_generic_path():
    from efficientgpt_amd.int8_linear import int8_matmul
    x, q, s = make_case(2, 2051, 33, seed=4)
    big = torch.zeros(2, 2051 + 3, dtype=torch.bfloat16)
    big[:, 3:] = x
    xd = big.cuda()[:, 3:]  # 6-byte offset rows: not 16-byte aligned
    y = int8_matmul(xd, q.cuda(), s.cuda())
    check_against_oracle(y, x, q, s)


def test_more_than_16_rows_refused_by_kernel():
    from efficientgpt_amd.int8_linear import int8_matmul
    q = torch.zeros(64, 32, device='cuda', dtype=torch.int8)
    with pytest.raises(ValueError):
        int8_matmul(torch.zeros(17, 32, device='cuda', dtype=torch.bfloat16), q, torch.ones(64, device='cuda'))
    with pytest.raises(ValueError):
        from efficientgpt_amd.int8_linear import int8_linear
        int8_linear(torch.zeros(1, 32, device='cuda'), q, torch.ones(64, device='cuda'))


def test_deterministic_and_inputs_untouched():
    from efficientgpt_amd.int8_linear import int8_linear
    x, q, s = make_case(1, 2048, 6144, seed=9)
    xd, qd, sd = x.cuda(), q.cuda(), s.cuda()
    xc, qc, sc = xd.clone(), qd.clone(), sd.clone()
    a = int8_linear(xd, qd, sd)
    b = int8_linear(xd, qd, sd)
    assert torch.equal(a, b)
    assert torch.equal(xd, xc) and torch.equal(qd, qc) and torch.equal(sd, sc)


def test_quantize_model_surgery():
    from efficientgpt_amd.int8_linear import Int8Linear, quantize_model
    torch.manual_seed(0)
    net = torch.nn.Sequential(torch.nn.Linear(128, 64, bias=True), torch.nn.GELU(), torch.nn.Linear(64, 32)).cuda()
    net = net.to(torch.bfloat16)
    x = torch.randn(5, 128, device='cuda', dtype=torch.bfloat16)
    ref = net(x).float()
    assert quantize_model(net, include_lm_head=False) == 2
    assert isinstance(net[0], Int8Linear)
    assert float((net(x).float() - ref).abs().max()) < 0.05 * float(ref.abs().max()) + 1e-2


def test_graph_capture_replay_bit_equal():
    from efficientgpt_amd.int8_linear import int8_linear
    q = torch.randint(-127, 128, (512, 256), device='cuda', dtype=torch.int8)
    s = torch.rand(512, device='cuda') * 0.01
    x = torch.randn(2, 256, device='cuda', dtype=torch.bfloat16)
    static_x = x.clone()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        int8_linear(static_x, q, s)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = int8_linear(static_x, q, s)
    for i in range(3):  # several replays, eager work between them
        static_x.copy_(x * (i + 2))
        g.replay()
        eager = int8_linear(x * (i + 2), q, s)
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


@pytest.mark.parametrize('k,n', [(2048, 6144), (6144, 2048), (2048, 4096), (1024, 100), (12288, 4096), (2064, 48)])
def test_single_row_matches_row_kernel_bitwise(k, n):
    """One aligned row goes to the fused kernel's store variant; the split-K entry with one split runs
    gemv_i8_rows and adds its single partial to zero. Both sum each lane's 1 KiB chunks in K order, remove
    128 * sum(x) once and reduce the row in the same fixed order, so the outputs must be bit-identical."""
    from efficientgpt_amd import _lib
    from efficientgpt_amd.int8_linear import int8_matmul
    x, q, s = make_case(1, k, n, seed=k + n)
    x, q, s = x.cuda(), q.cuda(), s.cuda()
    one = int8_matmul(x, q, s)
    ref = torch.empty_like(one)
    ws = torch.empty(max(4 * n, 4), device='cuda', dtype=torch.uint8)
    _lib.check('egpt_int8_gemv_splitk', _lib.lib().egpt_int8_gemv_splitk(
        x.data_ptr(), k, q.data_ptr(), k, s.data_ptr(), ref.data_ptr(), n, 1, n, k, 1, ws.data_ptr(), ws.numel(),
        _lib.stream_ptr()))
    assert torch.equal(one, ref)
    check_against_oracle(one.cpu(), x.cpu(), q.cpu(), s.cpu())


@pytest.mark.parametrize('m', [2, 3, 4])
@pytest.mark.parametrize('k,n', [(2048, 4096), (2048, 2048), (2048, 12288), (6144, 2048), (12288, 4096), (12288, 2048),
                                 (2064, 48), (1024, 100), (16, 7)])
def test_few_rows_equal_one_row_calls_bitwise(m, k, n):
    """Two aligned rows, and 3-4 rows under 4096 features, take the few-rows kernel: the one-row kernel's
    weight stream with the activation rows in LDS. Each row's chunk sums and row reduction run in the one-row
    kernel's order, so each output row must equal a one-row call on that row bit for bit; with strided rows
    (ldx > K, ldy > N) too. 3-4 rows over 4096 features or more take the MFMA kernel: oracle check only."""
    from efficientgpt_amd import _lib
    from efficientgpt_amd.int8_linear import int8_matmul
    x, q, s = make_case(m, k, n, seed=k * 3 + n + m)
    xd, qd, sd = x.cuda(), q.cuda(), s.cuda()
    few = int8_matmul(xd, qd, sd)
    check_against_oracle(few.cpu(), x, q, s)
    if m > 2 and n >= 4096:
        return
    ones = torch.cat([int8_matmul(xd[i:i + 1].contiguous(), qd, sd) for i in range(m)])
    assert torch.equal(few, ones)
    # strided rows: x rows 2k + 16 apart, y rows n + 5 apart
    xs = torch.zeros(m, 2 * k + 16, dtype=torch.bfloat16, device='cuda')
    xs[:, :k] = xd
    ys = torch.full((m, n + 5), 7.0, dtype=torch.bfloat16, device='cuda')
    _lib.check('egpt_int8_gemv', _lib.lib().egpt_int8_gemv(xs.data_ptr(), xs.stride(0), qd.data_ptr(), k,
                                                             sd.data_ptr(), ys.data_ptr(), ys.stride(0), m, n, k,
                                                             _lib.stream_ptr()))
    torch.cuda.synchronize()
    assert torch.equal(ys[:, :n], few)
    assert bool((ys[:, n:] == 7.0).all())  # nothing written past N


@pytest.mark.parametrize('m', [3, 4, 8, 16])
@pytest.mark.parametrize('k,n', [(2048, 4096), (6144, 2048), (2048, 100), (12288, 48), (512, 32768), (1024, 70001),
                                 (2048, 12288), (2048, 65600), (1536, 20000), (4096, 12000), (6144, 9000)])
def test_small_batch_mfma_kernel_matches_oracle(m, k, n):
    """3-16 rows take the MFMA kernel (K a multiple of 64, aligned rows; 3-4 rows under 4096 features the
    few-rows kernel): against the oracle's decode rule, odd N, the longest K, 2048 feature groups (32768
    features), and an odd width past 65536 features, where each wavefront serves four groups of 16. Past 8192
    features with K <= 2048 the blocks walk tiles; for K of 1024-2048 in 512-byte chunks the weights are staged
    through LDS (12288 x 2048, 20000 x 1536, 12000 x 4096 and 9000 x 6144 with one group per tile, 65600 x 2048
    and 70001 x 1024 with four, a ragged last tile), at K = 512 they go to registers (32768 x 512)."""
    from efficientgpt_amd.int8_linear import int8_matmul
    x, q, s = make_case(m, k, n, seed=100 + m + k + n)
    xd, qd, sd = x.cuda(), q.cuda(), s.cuda()
    y = int8_matmul(xd, qd, sd)
    check_against_oracle(y.cpu(), x, q, s)
    again = int8_matmul(xd, qd, sd)
    assert torch.equal(y, again)  # fixed reduction order: reproducible


def test_small_batch_lds_kernel_four_groups_long_rows():
    """8 rows over 65600 x 3072: the LDS-staged MFMA GEMV with four feature groups per tile and six 512-byte
    chunks per row, a ragged last tile; against the oracle, reproducible."""
    from efficientgpt_amd.int8_linear import int8_matmul
    x, q, s = make_case(8, 3072, 65600, seed=77)
    xd, qd, sd = x.cuda(), q.cuda(), s.cuda()
    y = int8_matmul(xd, qd, sd)
    check_against_oracle(y.cpu(), x, q, s)
    assert torch.equal(y, int8_matmul(xd, qd, sd))


PREFILL_SHAPES = [(17, 64, 64), (33, 2048, 4096), (128, 2048, 4096), (100, 2048, 6144), (300, 6144, 2048),
                  (1000, 1024, 96), (257, 4096, 1000), (4096, 2048, 2048), (300, 192, 4096), (4096, 128, 4096),
                  (2100, 704, 4000), (2304, 320, 7424), (1000, 448, 4100), (1024, 512, 2048), (1000, 320, 2100),
                  (200, 2048, 2048), (130, 2048, 2100), (250, 6144, 2048), (4096, 64, 4096), (4100, 192, 4000)]


@pytest.mark.parametrize('m,k,n', PREFILL_SHAPES)
def test_prefill_gemm_kernel_matches_oracle(m, k, n):
    """More than 16 rows: the MFMA GEMM (egpt_int8_gemm), against the oracle's prefill formula
    bf16(fp32(bf16(x q^T)) s) and the reference's tolerance; odd N and M exercise the masked edges,
    K = 192 an odd number of 64-wide K steps; 4096 x 2048 -> 2048 and 2100 x 704 -> 4000 (ragged) take the
    128 x 256 tile, 4096 x 128 -> 4096, 2304 x 320 -> 7424 (5 K steps), 4096 x 64 -> 4096 (one K step) and
    4100 x 192 -> 4000 (ragged M and N) the 256 x 256 tile whose operands go straight into LDS,
    1000 x 448 -> 4100 the 8-wavefront 128 x 128 tile, 1024 x 512 -> 2048 and 1000 x 320 -> 2100 (ragged) the
    128 x 64 tile; every tile with two wavefronts along M takes its weights into LDS as bf16. 200 x 2048 -> 2048,
    130 x 2048 -> 2100 (ragged) and 250 x 6144 -> 2048 are 64 x 64 grids with fewer tiles than CUs, which take
    128-wide K steps."""
    from efficientgpt_amd import _lib
    x, q, s = make_case(m, k, n, seed=m + k + n)
    xd, qd, sd = x.cuda(), q.cuda(), s.cuda()
    y = torch.empty(m, n, device='cuda', dtype=torch.bfloat16)
    st = _lib.lib().egpt_int8_gemm(xd.data_ptr(), k, qd.data_ptr(), k, sd.data_ptr(), y.data_ptr(), n, m, n, k,
                                   _lib.stream_ptr())
    assert st == 0, st  # aligned shapes take the kernel, not the library formula
    check_against_oracle(y.cpu(), x, q, s)
    lib_form = ((xd @ qd.to(torch.bfloat16).t()).float() * sd).to(torch.bfloat16)
    diff = (y.float() - lib_form.float()).abs()
    assert float((diff == 0).float().mean()) >= 0.9


SPLIT_SHAPES = [(128, 6144, 2048), (128, 2048, 4096), (33, 6144, 2048), (64, 2048, 2048), (100, 4096, 1000),
                (17, 12288, 64), (200, 2048, 2048), (130, 2048, 2000), (256, 2048, 2048)]


@pytest.mark.parametrize('m,k,n', SPLIT_SHAPES)
def test_prefill_gemm_split_k_matches_oracle(m, k, n):
    """Short-M shapes whose 64 x 64 tiles leave CUs idle split K through a workspace (egpt_int8_gemm_ws; past 128
    rows, up to 256, grids of at most 128 tiles): the splits' fp32 tiles are added in order, then rounded as the
    reference's formula. Same bounds as the one-pass
    kernel, and the same result as it on all but the elements whose fp32 sum rounds differently."""
    from efficientgpt_amd import _lib
    import ctypes
    lib = _lib.lib()
    need = ctypes.c_size_t()
    assert lib.egpt_int8_gemm_workspace(m, n, k, ctypes.byref(need)) == 0
    assert need.value > 0 and need.value % (m * n * 4) == 0, need.value
    x, q, s = make_case(m, k, n, seed=m + k + n)
    xd, qd, sd = x.cuda(), q.cuda(), s.cuda()
    ws = torch.empty(need.value, device='cuda', dtype=torch.uint8)
    y = torch.empty(m, n, device='cuda', dtype=torch.bfloat16)
    st = lib.egpt_int8_gemm_ws(xd.data_ptr(), k, qd.data_ptr(), k, sd.data_ptr(), y.data_ptr(), n, m, n, k,
                               ws.data_ptr(), need.value, _lib.stream_ptr())
    assert st == 0, st
    check_against_oracle(y.cpu(), x, q, s)
    one = torch.empty_like(y)
    assert lib.egpt_int8_gemm(xd.data_ptr(), k, qd.data_ptr(), k, sd.data_ptr(), one.data_ptr(), n, m, n, k,
                              _lib.stream_ptr()) == 0
    assert float((one == y).float().mean()) >= 0.9
    # too small a workspace is refused before any launch
    assert lib.egpt_int8_gemm_ws(xd.data_ptr(), k, qd.data_ptr(), k, sd.data_ptr(), y.data_ptr(), n, m, n, k,
                                 ws.data_ptr(), need.value - 4, _lib.stream_ptr()) == -4
    # the op takes the split path and reproduces it bit for bit
    from efficientgpt_amd.int8_linear import int8_linear
    assert torch.equal(int8_linear(xd, qd, sd), y)


GENERIC_SHAPES = [(40, 100, 70), (17, 2051, 33), (64, 96, 257)]


@pytest.mark.parametrize('m,k,n', GENERIC_SHAPES)
def test_prefill_generic_kernel_for_shapes_the_mfma_kernel_refuses(m, k, n):
    """K not a multiple of 64, and x rows 6 bytes off 16-byte alignment: egpt_int8_gemm runs its generic
    kernel (no library formula anywhere in the op) with the prefill formula's two roundings, against the oracle."""
    from efficientgpt_amd import _lib
    from efficientgpt_amd.int8_linear import int8_linear
    x, q, s = make_case(m, k, n, seed=m + k + n)
    qd, sd = q.cuda(), s.cuda()
    big = torch.zeros(m, k + 3, dtype=torch.bfloat16)
    big[:, 3:] = x
    xd = big.cuda()[:, 3:]  # unaligned rows, row stride k + 3
    y = torch.full((m, n), float('nan'), device='cuda', dtype=torch.bfloat16)
    st = _lib.lib().egpt_int8_gemm(xd.data_ptr(), k + 3, qd.data_ptr(), k, sd.data_ptr(), y.data_ptr(), n, m, n, k,
                                   _lib.stream_ptr())
    assert st == 0, st
    check_against_oracle(y.cpu(), x, q, s)
    assert torch.equal(int8_linear(xd, qd, sd), y)  # the op takes the same kernel


def test_prefill_op_keeps_leading_dims():
    from efficientgpt_amd.int8_linear import int8_linear
    x, q, s = make_case(48, 2048, 512, seed=11)
    y = int8_linear(x.cuda().view(4, 12, 2048), q.cuda(), s.cuda())  # leading dims, kernel path
    assert y.shape == (4, 12, 512)
    check_against_oracle(y.view(48, 512).cpu(), x, q, s)


@pytest.mark.parametrize('rows', [1, 3, 40])
def test_int8_linear_opcheck(rows):
    """torch.library.opcheck of efficientgpt::int8_linear on device tensors: schema, fake implementation
    (shape / dtype / device against the real kernel's output) and AOT dispatch, at decode (1, 3 rows: the GEMV)
    and prefill (40 rows: the GEMM) sizes. The reference pins its fake through torch.compile parity
    (research/realmodel/test_int8_linear.py:62-79)."""
    g = torch.Generator().manual_seed(rows)
    x = torch.randn(rows, 2048, generator=g).to(torch.bfloat16).cuda()
    w = torch.randint(-127, 128, (512, 2048), generator=g, dtype=torch.int8).cuda()
    s = (torch.rand(512, generator=g) * 0.01 + 1e-3).cuda()
    torch.library.opcheck(torch.ops.efficientgpt.int8_linear.default, (x, w, s))


@pytest.mark.parametrize('m,k,n', [(128, 6144, 2048), (128, 2048, 2048), (64, 2048, 2048), (33, 6144, 2048),
                                   (100, 4096, 1000)])
def test_gemm_add_rmsnorm_matches_the_two_calls_bit_for_bit(m, k, n):
    """egpt_int8_gemm_add_rmsnorm (split slices, then one row kernel: the splits' sum, both roundings, the residual
    and the RMSNorm) against egpt_int8_gemm_ws followed by egpt_add_rmsnorm on the same inputs: residual and norm
    output bit-identical; too small a workspace and unsplit shapes are refused before any launch."""
    from efficientgpt_amd import _lib
    import ctypes
    lib = _lib.lib()
    need = ctypes.c_size_t()
    assert lib.egpt_int8_gemm_workspace(m, n, k, ctypes.byref(need)) == 0 and need.value > 0
    x, q, s = make_case(m, k, n, seed=3 * m + n)
    xd, qd, sd = x.cuda(), q.cuda(), s.cuda()
    g = torch.Generator().manual_seed(m + k)
    resid = torch.randn(m, n, generator=g).to(torch.bfloat16).cuda()
    nw = (1 + 0.1 * torch.randn(n, generator=g)).to(torch.bfloat16).cuda()
    ws = torch.empty(need.value, device='cuda', dtype=torch.uint8)
    st = _lib.stream_ptr()
    # two calls
    o = torch.empty(m, n, device='cuda', dtype=torch.bfloat16)
    r2, h2 = resid.clone(), torch.empty(m, n, device='cuda', dtype=torch.bfloat16)
    assert lib.egpt_int8_gemm_ws(xd.data_ptr(), k, qd.data_ptr(), k, sd.data_ptr(), o.data_ptr(), n, m, n, k,
                                 ws.data_ptr(), need.value, st) == 0
    assert lib.egpt_add_rmsnorm(r2.data_ptr(), n, o.data_ptr(), n, nw.data_ptr(), h2.data_ptr(), n, m, n, 1e-6, st) == 0
    # one call
    r1, h1 = resid.clone(), torch.full((m, n), float('nan'), device='cuda', dtype=torch.bfloat16)
    assert lib.egpt_int8_gemm_add_rmsnorm(xd.data_ptr(), k, qd.data_ptr(), k, sd.data_ptr(), r1.data_ptr(), n,
                                          nw.data_ptr(), h1.data_ptr(), n, m, n, k, 1e-6, ws.data_ptr(), need.value,
                                          st) == 0
    torch.cuda.synchronize()
    assert torch.equal(r1, r2) and torch.equal(h1, h2)
    assert not bool(torch.isnan(h1.float()).any())
    assert lib.egpt_int8_gemm_add_rmsnorm(xd.data_ptr(), k, qd.data_ptr(), k, sd.data_ptr(), r1.data_ptr(), n,
                                          nw.data_ptr(), h1.data_ptr(), n, m, n, k, 1e-6, ws.data_ptr(),
                                          need.value - 4, st) == _lib.EGPT_ERR_WORKSPACE
    assert lib.egpt_int8_gemm_add_rmsnorm(xd.data_ptr(), k, qd.data_ptr(), k, sd.data_ptr(), r1.data_ptr(), n,
                                          nw.data_ptr(), h1.data_ptr(), n, 1024, n, k, 1e-6, ws.data_ptr(),
                                          need.value, st) == _lib.EGPT_ERR_UNSUPPORTED  # 1024 rows: K not split


@pytest.mark.parametrize('m,k,inter', [(1024, 2048, 6144), (2048, 4096, 12288), (1100, 512, 7000), (128, 2048, 6144),
                                        (100, 2048, 6144), (200, 2048, 6144), (130, 512, 7000), (40, 4096, 12288),
                                        (2048, 192, 4200)])
def test_gemm_swiglu_matches_the_two_calls_bit_for_bit(m, k, inter):
    """egpt_int8_gemm_swiglu (SwiGLU in the epilogue of the gate/up product, the gate and up rows of a feature
    paired in one wavefront: two column tiles of its large tiles, or the two halves of its one 64 x 64 tile)
    against egpt_int8_gemm into a [m, 2 inter] buffer followed by egpt_silu_mul: the same bits, ragged rows and
    features included; a shape whose plain product would split K is refused."""
    from efficientgpt_amd import _lib
    lib = _lib.lib()
    x, q, s = make_case(m, k, 2 * inter, seed=m + inter)
    xd, qd, sd = x.cuda(), q.cuda(), s.cuda()
    st = _lib.stream_ptr()
    gu = torch.empty(m, 2 * inter, device='cuda', dtype=torch.bfloat16)
    assert lib.egpt_int8_gemm(xd.data_ptr(), k, qd.data_ptr(), k, sd.data_ptr(), gu.data_ptr(), 2 * inter, m,
                              2 * inter, k, st) == 0
    two = torch.empty(m, inter, device='cuda', dtype=torch.bfloat16)
    assert lib.egpt_silu_mul(gu.data_ptr(), 2 * inter, inter, two.data_ptr(), inter, m, st) == 0
    one = torch.full((m, inter), float('nan'), device='cuda', dtype=torch.bfloat16)
    assert lib.egpt_int8_gemm_swiglu(xd.data_ptr(), k, qd.data_ptr(), k, sd.data_ptr(), one.data_ptr(), inter, m,
                                     inter, k, st) == 0
    torch.cuda.synchronize()
    assert torch.equal(one, two)
    # 64 rows over 1024 features: the plain product's 32 tiles split K where K is a multiple of the 128-wide split
    # step (refused), and run unsplit otherwise
    expect = _lib.EGPT_ERR_UNSUPPORTED if k % 128 == 0 else 0
    assert lib.egpt_int8_gemm_swiglu(xd.data_ptr(), k, qd.data_ptr(), k, sd.data_ptr(), one.data_ptr(), inter, 64,
                                     1024, k, st) == expect

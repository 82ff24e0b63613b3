"""Parity of each HIP kernel with the oracle on the same seeded inputs (through the C ABI).

Bars: bit-exact for Q8_0 dequantisation, repacking, activation quantisation, the Q8_0 GEMV/GEMM
(the device reproduces ggml-cpu's x86 summation order), the F16/F32 head dots and the
LayerNorm; attention within 2e-3 relative (max |diff| / max |ref|), fp32 accumulation over an
fp16 cache.
"""
import numpy as np
import pytest

import oracle as O
import synth_model as sm

pytestmark = pytest.mark.gpu


def _dev(a, torch):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def unslice(qs: np.ndarray, k: int) -> np.ndarray:
    """sliced [rows][8][nblk][4] -> natural [rows][k] int8"""
    rows = qs.size // k
    return qs.reshape(rows, 8, k // 32, 4).transpose(0, 2, 1, 3).reshape(rows, k)


def to_tiled(q: np.ndarray, d: np.ndarray):
    """Quants [R][K] and scales [R][K/32] in the matrix-core operand order: per 32-row tile and
    block, 1 KB where bytes [16L, 16L+16), L = 32h + i, are quants [16h, 16h+16) of row i; the
    tile's 32 scales of the block in row order. Rows padded to 32 with zeros."""
    R, K = q.shape
    nb, Rp = K // 32, (R + 31) // 32 * 32
    qp = np.zeros((Rp, K), q.dtype)
    qp[:R] = q
    dp = np.zeros((Rp, nb), d.dtype)
    dp[:R] = d
    qt = qp.reshape(Rp // 32, 32, nb, 2, 16).transpose(0, 2, 3, 1, 4).reshape(-1)
    dt = dp.reshape(Rp // 32, 32, nb).transpose(0, 2, 1).reshape(-1)
    return np.ascontiguousarray(qt), np.ascontiguousarray(dt)


def blocks_to_split(blocks: np.ndarray, rows: int, k: int):
    b = blocks.reshape(rows, k // 32, 34)
    d = b[:, :, 0:2].copy().view(np.uint16)[:, :, 0]
    q = b[:, :, 2:].view(np.int8).reshape(rows, k)
    return q, d


def _special_rows(rng, k):
    x = rng.standard_normal((6, k)).astype(np.float32)
    x[0, :32] = 0.0                                     # all-zero block: d = 0, q = 0
    x[1, :32] = -0.0                                    # negative zeros
    x[2, :32] = np.linspace(-1, 1, 32)                  # +-amax extremes -> +-127
    x[3, :32] = 0.5                                     # constant block
    x[4, :32] = np.float32(1e-30)                       # subnormal-range scale
    x[5, :32] = (np.arange(32) - 15.5).astype(np.float32) / 127.0 * 4  # exact .5 ties at id=127/amax
    return x


def test_q8_dequant_bitexact(gpu):
    import torch
    rng = np.random.default_rng(1)
    x = np.concatenate([_special_rows(rng, 512), rng.standard_normal((64, 512)).astype(np.float32) * 0.02])
    blocks = sm.q8_quantize_ref(x).ravel()
    out = torch.zeros(x.size, dtype=torch.float32, device="cuda")
    gpu.op_q8_dequant(_dev(blocks, torch), out)
    torch.cuda.synchronize()
    ref = O.q8_dequant(blocks)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), ref.view(np.uint32))


def test_q8_repack_bitexact(gpu):
    import torch
    rng = np.random.default_rng(2)
    rows, k = 40, 2048
    blocks = sm.q8_quantize_ref(rng.standard_normal((rows, k)).astype(np.float32) * 0.02).ravel()
    qs = torch.zeros(rows * k, dtype=torch.int8, device="cuda")
    d = torch.zeros(rows * k // 32, dtype=torch.int16, device="cuda")
    gpu.op_q8_repack(_dev(blocks, torch), rows, k, qs, d)
    torch.cuda.synchronize()
    q_ref, d_ref = blocks_to_split(blocks, rows, k)
    assert np.array_equal(unslice(qs.cpu().numpy(), k), q_ref)
    assert np.array_equal(d.cpu().numpy().view(np.uint16).reshape(rows, -1), d_ref)


@pytest.mark.parametrize("k", [512, 2048])
def test_q8_quantize_bitexact(gpu, k):
    import torch
    rng = np.random.default_rng(3 + k)
    x = np.concatenate([_special_rows(rng, k), rng.standard_normal((97, k)).astype(np.float32) * 3.0])
    rows = x.shape[0]
    xq = torch.zeros(rows * k, dtype=torch.int8, device="cuda")
    xd = torch.zeros(rows * k // 32, dtype=torch.float32, device="cuda")
    gpu.op_q8_quantize(_dev(x, torch), xq, xd)
    torch.cuda.synchronize()
    ref = O.q8_quantize_x86(x)
    q_ref, d_ref = blocks_to_split(ref, rows, k)
    assert np.array_equal(unslice(xq.cpu().numpy(), k), q_ref)
    d_ref32 = d_ref.view(np.float16).astype(np.float32)
    assert np.array_equal(xd.cpu().numpy().reshape(rows, -1).view(np.uint32), d_ref32.view(np.uint32))


@pytest.mark.parametrize("n,k", [(1536, 512), (512, 512), (2048, 512), (512, 2048)])
@pytest.mark.parametrize("m", [1, 4, 16, 37, 64, 300])
def test_q8_gemv_bitexact(gpu, n, k, m):
    import torch
    rng = np.random.default_rng(n * 7 + k + m)
    W = rng.standard_normal((n, k)).astype(np.float32) * 0.02
    X = rng.standard_normal((m, k)).astype(np.float32)
    X[0, :64] = 0.0
    wb = sm.q8_quantize_ref(W).ravel()
    wq = torch.zeros(n * k, dtype=torch.int8, device="cuda")
    wd = torch.zeros(n * k // 32, dtype=torch.int16, device="cuda")
    gpu.op_q8_repack(_dev(wb, torch), n, k, wq, wd)
    xq = torch.zeros(m * k, dtype=torch.int8, device="cuda")
    xd = torch.zeros(m * k // 32, dtype=torch.float32, device="cuda")
    gpu.op_q8_quantize(_dev(X, torch), xq, xd)
    y = torch.zeros((m, n), dtype=torch.float32, device="cuda")
    gpu.op_q8_gemv(wq, wd, n, k, xq, xd, m, None, 0, y)
    bias = rng.standard_normal(n).astype(np.float32) * 0.02
    y2 = torch.zeros((m, n), dtype=torch.float32, device="cuda")
    gpu.op_q8_gemv(wq, wd, n, k, xq, xd, m, _dev(bias, torch), 1, y2)
    torch.cuda.synchronize()
    ref = O.q8_matmul(wb, n, k, X)
    got = y.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), \
        f"max |diff| {np.abs(got - ref).max():.3e}, mismatches {(got != ref).sum()}"
    ref2 = np.maximum(ref + bias[None, :], 0.0).astype(np.float32)
    assert np.array_equal(y2.cpu().numpy(), ref2)


@pytest.mark.parametrize("n", [1536, 2048])
@pytest.mark.parametrize("m", [1, 16, 41])
def test_ln_gemv_bitexact(gpu, n, m):
    """The fused LayerNorm -> Q8_0 -> GEMV kernel equals LayerNorm, x86 quantisation and the
    Q8_0 dot of the oracle, to the bit."""
    import torch
    rng = np.random.default_rng(n + m)
    k = 512
    W = rng.standard_normal((n, k)).astype(np.float32) * 0.02
    res = rng.standard_normal((m, k)).astype(np.float32)
    r = rng.standard_normal((m, k)).astype(np.float32) * 0.5
    lb = rng.standard_normal(k).astype(np.float32) * 0.02
    wb = np.concatenate([1 + 0.05 * rng.standard_normal(k), 0.05 * rng.standard_normal(k)]).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32) * 0.02
    wbk = sm.q8_quantize_ref(W).ravel()
    wq = torch.zeros(n * k, dtype=torch.int8, device="cuda")
    wd = torch.zeros(n * k // 32, dtype=torch.int16, device="cuda")
    gpu.op_q8_repack(_dev(wbk, torch), n, k, wq, wd)
    y = torch.zeros((m, n), dtype=torch.float32, device="cuda")
    ln = torch.zeros((m, k), dtype=torch.float32, device="cuda")
    gpu.op_ln_gemv(wq, wd, n, _dev(res, torch), _dev(r, torch), _dev(lb, torch), _dev(wb, torch),
                   _dev(bias, torch), 1, y, ln_out=ln)
    torch.cuda.synchronize()
    ln_ref = O.layernorm(res, r, lb, wb)
    assert np.array_equal(ln.cpu().numpy(), ln_ref)
    ref = np.maximum(O.q8_matmul(wbk, n, k, ln_ref) + bias[None, :], 0.0).astype(np.float32)
    assert np.array_equal(y.cpu().numpy(), ref)


@pytest.mark.parametrize("rows,n", [(1, 512), (16, 512), (333, 512), (8, 1024)])
def test_layernorm(gpu, rows, n):
    import torch
    rng = np.random.default_rng(rows + n)
    x = rng.standard_normal((rows, n)).astype(np.float32) * 2 + 0.3
    r = rng.standard_normal((rows, n)).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32) * 0.1
    wb = np.concatenate([1 + 0.1 * rng.standard_normal(n), 0.1 * rng.standard_normal(n)]).astype(np.float32)
    y = torch.zeros((rows, n), dtype=torch.float32, device="cuda")
    yq = torch.zeros(rows * n, dtype=torch.int8, device="cuda")
    yd = torch.zeros(rows * n // 32, dtype=torch.float32, device="cuda")
    gpu.op_layernorm(_dev(x, torch), _dev(r, torch), _dev(bias, torch), _dev(wb, torch), 1e-5, y, yq, yd)
    y0 = torch.zeros((rows, n), dtype=torch.float32, device="cuda")
    gpu.op_layernorm(_dev(x, torch), None, None, _dev(wb, torch), 1e-5, y0)
    torch.cuda.synchronize()
    ref = O.layernorm(x, r, bias, wb)
    got = y.cpu().numpy()
    # sums are in double on both sides (only their order differs): equal to the bit
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), f"max {np.abs(got - ref).max():.3e}"
    assert np.array_equal(y0.cpu().numpy(), O.layernorm(x, None, None, wb))
    q_ref, d_ref = blocks_to_split(O.q8_quantize_x86(ref), rows, n)
    assert np.array_equal(unslice(yq.cpu().numpy(), n), q_ref)
    assert np.array_equal(yd.cpu().numpy().reshape(rows, -1), d_ref.view(np.float16).astype(np.float32))


def _ref_act(v, act):
    import math
    v = v.astype(np.float64)
    if act == 1:
        return np.maximum(v, 0)
    if act == 2:
        return 0.5 * v * (1 + np.vectorize(math.erf)(v / math.sqrt(2)))
    if act == 3:
        return v * np.tanh(np.log1p(np.exp(v)))
    return v


@pytest.mark.parametrize("act", [0, 1, 2, 3])
def test_add_act_reference_fixture(gpu, act):
    """tests/test_add_act.cpp:66-101: a[i] = 0.02*((i*37 % 101) - 50) + 0.5, b[i] =
    0.01*((i*13 % 29) - 14), NE0 = 64, NR = 7; tolerance 2e-3 (5e-3 for GELU)."""
    import torch
    NE0, NR = 64, 7
    i = np.arange(NE0 * NR)
    a = (0.02 * ((i * 37 % 101) - 50) + 0.5).astype(np.float32)
    j = np.arange(NE0)
    b = (0.01 * ((j * 13) % 29 - 14)).astype(np.float32)
    y = torch.zeros(NE0 * NR, dtype=torch.float32, device="cuda")
    gpu.op_add_act(_dev(a, torch), _dev(b, torch), act, y)
    torch.cuda.synchronize()
    ref = _ref_act((a.reshape(NR, NE0) + b).ravel(), act)
    tol = 5e-3 if act == 2 else 2e-3
    assert np.abs(y.cpu().numpy() - ref).max() <= tol
    if act in (0, 1):
        assert np.array_equal(y.cpu().numpy(), O.add_act(a, b, act))


@pytest.mark.parametrize("wtype", [0, 1])
@pytest.mark.parametrize("mode", [0, 1])
def test_fdot_head_bitexact(gpu, wtype, mode):
    import torch
    rng = np.random.default_rng(10 + wtype * 2 + mode)
    n, k, m = 1025, 512, 5
    W = rng.standard_normal((n, k)).astype(np.float32) * 0.02
    X = rng.standard_normal((m, k)).astype(np.float32)
    y = torch.zeros((m, n), dtype=torch.float32, device="cuda")
    if wtype == 1:
        W16 = W.astype(np.float16).view(np.uint16)
        gpu.op_fdot(_dev(W16, torch), 1, _dev(X, torch), y, mode)
        ref = O.f16_matmul(W16, X, mode)
    else:
        gpu.op_fdot(_dev(W, torch), 0, _dev(X, torch), y, mode)
        ref = O.f32_matmul(W, X, mode)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), f"max {np.abs(got - ref).max():.3e}"


@pytest.mark.parametrize("m,k,n", [(9, 1025, 512), (70, 1025, 512), (333, 1025, 512), (2050, 1025, 512),
                                   (96, 1024, 512), (130, 1025, 200)])
def test_fdot_bert_projection_bitexact(gpu, m, k, n):
    """K = 1025 (bert_aug = [W | b]): ggml_vec_dot_f32 with a fused leftover. From 64 rows, n % 32
    == 0: the fp32 matrix-core kernel (one product per instruction and output, the same chains);
    n = 200: the kernel that keeps 4 weight rows x 16 activation rows per thread."""
    import torch
    rng = np.random.default_rng(20 + m + k + n)
    W = rng.standard_normal((n, k)).astype(np.float32) * 0.02
    X = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    X[:, k - 1] = 1.0
    y = torch.zeros((m, n), dtype=torch.float32, device="cuda")
    gpu.op_fdot(_dev(W, torch), 0, _dev(X, torch), y, 0)
    torch.cuda.synchronize()
    ref = O.f32_matmul(W, X, 0)
    assert np.array_equal(y.cpu().numpy(), ref)


def _attn_case(rng, B, nh, lstride, begins, ends):
    q = rng.standard_normal((B, nh, 32)).astype(np.float32)
    k = rng.standard_normal((B, nh, lstride, 32)).astype(np.float16).view(np.uint16)
    v = rng.standard_normal((B, nh, lstride, 32)).astype(np.float16).view(np.uint16)
    return q, k, v, np.asarray(begins, np.int32), np.asarray(ends, np.int32)


def _run_attn(gpu, torch, q, k, v, kb, ke, max_keys, quant=False):
    B, nh, _ = q.shape
    scale = np.float32(1.0) / np.sqrt(np.float32(32.0))
    out = torch.zeros((B, nh * 32), dtype=torch.float32, device="cuda")
    ws = torch.zeros(gpu.attn_workspace_bytes(B, nh, max_keys), dtype=torch.uint8, device="cuda")
    oq = torch.zeros(B * nh * 32, dtype=torch.int8, device="cuda") if quant else None
    od = torch.zeros(B * nh, dtype=torch.float32, device="cuda") if quant else None
    args = [_dev(q, torch), _dev(k, torch), _dev(v, torch), _dev(kb, torch), _dev(ke, torch), max_keys,
            float(scale), out]
    gpu.op_attn_decode(*args, oq=oq, od=od, ws=ws)
    torch.cuda.synchronize()
    first = out.cpu().numpy().copy()
    gpu.op_attn_decode(*args, oq=oq, od=od, ws=ws)       # counters must have been reset
    torch.cuda.synchronize()
    assert np.array_equal(first, out.cpu().numpy())
    return first, scale, (None if not quant else (oq.cpu().numpy(), od.cpu().numpy()))


def test_attn_decode_parity(gpu):
    import torch
    rng = np.random.default_rng(30)
    B, nh, lstride = 12, 16, 1100
    begins = rng.integers(0, 200, B)
    ends = np.minimum(lstride, begins + rng.integers(1, 900, B))
    begins[0], ends[0] = 0, 1           # one key: output = that V row
    begins[1], ends[1] = 5, 5 + 256     # exactly one chunk
    begins[2], ends[2] = 3, 3 + 257     # one key into the second chunk
    begins[3], ends[3] = 0, lstride     # the whole cache
    q, k, v, kb, ke = _attn_case(rng, B, nh, lstride, begins, ends)
    got, scale, qd = _run_attn(gpu, torch, q, k, v, kb, ke, lstride, quant=True)
    ref = O.attn_decode_f16(q, k, v, kb, ke, scale)
    rel = np.abs(got - ref).max() / np.abs(ref).max()
    assert rel <= 2e-3, rel
    assert rel <= 1e-5, rel   # fp32 accumulation over the same fp16 data: far inside the bar
    v0 = v[0, :, 0, :].view(np.float16).astype(np.float32).reshape(-1)
    assert np.allclose(got[0], v0, rtol=0, atol=1e-6)
    # the Q8_0 copy is the x86 quantisation of the fp32 output (one block per head)
    q_ref, d_ref = blocks_to_split(O.q8_quantize_x86(got), B, nh * 32)
    assert np.array_equal(unslice(qd[0], nh * 32), q_ref)


@pytest.mark.parametrize("B,nh,lstride,what", [
    (8, 16, 200, "4 waves per workgroup (rows of at most 4 blocks)"),
    (4, 16, 400, "8 waves per workgroup"),
    (80, 16, 1000, "4 waves per workgroup (1280 (seq, head) pairs cap the grid)"),
    (40, 16, 1000, "8 waves per workgroup (640 pairs)"),
    (2, 4, 4096, "8 waves per workgroup, 4 splits merged by the last workgroup"),
    (1, 16, 3000, "8 waves per workgroup, 2 splits"),
    (64, 16, 3100, "4 waves, rows cut in chunks of 16 blocks (1024 pairs), merged by a second launch"),
])
def test_attn_decode_launch_shapes(gpu, B, nh, lstride, what):
    import torch
    rng = np.random.default_rng(33 + B)
    begins = rng.integers(0, lstride // 4, B)
    ends = np.minimum(lstride, begins + rng.integers(1, lstride, B))
    ends[-1] = lstride                    # one row reaches the end of the buffer
    if B > 2:
        ends[0] = begins[0]               # and one is empty
    q, k, v, kb, ke = _attn_case(rng, B, nh, lstride, begins, ends)
    got, scale, _ = _run_attn(gpu, torch, q, k, v, kb, ke, lstride)
    ref = O.attn_decode_f16(q, k, v, kb, ke, scale)
    assert np.abs(got - ref).max() / np.abs(ref).max() <= 1e-5, what
    if B > 2:
        assert np.all(got[0] == 0.0)


def test_attn_decode_rows_longer_than_planned(gpu):
    """Rows longer than max_keys (the length the launch is planned for: here 3 chunks of 16
    blocks) get longer runs per split instead of more splits; the output is unchanged."""
    import torch
    rng = np.random.default_rng(34)
    B, nh, lstride = 64, 16, 3700
    begins = rng.integers(0, 100, B)
    ends = np.minimum(lstride, begins + rng.integers(2000, lstride, B))
    ends[3] = lstride
    q, k, v, kb, ke = _attn_case(rng, B, nh, lstride, begins, ends)
    got, scale, _ = _run_attn(gpu, torch, q, k, v, kb, ke, 3072)
    ref = O.attn_decode_f16(q, k, v, kb, ke, scale)
    assert np.abs(got - ref).max() / np.abs(ref).max() <= 1e-5


def test_attn_decode_empty_and_constant(gpu):
    import torch
    rng = np.random.default_rng(31)
    B, nh, lstride = 3, 4, 600
    q, k, v, kb, ke = _attn_case(rng, B, nh, lstride, [7, 0, 10], [7, 600, 530])
    v[1] = np.float16(0.75).view(np.uint16)               # constant V -> output = V
    got, _, _ = _run_attn(gpu, torch, q, k, v, kb, ke, lstride)
    assert np.all(got[0] == 0.0)                          # no valid key -> 0 (ggml: S == 0)
    assert np.allclose(got[1], 0.75, rtol=0, atol=1e-6)


def test_attn_decode_microbench_shape(gpu):
    """The decode-attention microkernel configuration at its own shape and launch, as the
    benchmark times it: batch 64 x 16 heads x 32, one query per sequence, KV lengths uniform
    256-2048 from the benchmark's seed, fp16 K/V ~ N(0,1), planned for 2048 keys (one workgroup
    per (sequence, head), 8 waves, no split), fp32 output and its fp16 copy."""
    import torch
    rng = np.random.Generator(np.random.PCG64(0x6A5E0003))
    B, nh, lstride = 64, 16, 2048
    L = rng.integers(256, 2049, B)
    q, k, v, kb, ke = _attn_case(np.random.default_rng(32), B, nh, lstride, np.zeros(B), L)
    scale = np.float32(1.0) / np.sqrt(np.float32(32.0))
    out = torch.zeros((B, nh * 32), dtype=torch.float32, device="cuda")
    out16 = torch.zeros((B, nh * 32), dtype=torch.float16, device="cuda")
    ws = torch.zeros(gpu.attn_workspace_bytes(B, nh, lstride), dtype=torch.uint8, device="cuda")
    gpu.op_attn_decode(_dev(q, torch), _dev(k, torch), _dev(v, torch), _dev(kb, torch), _dev(ke, torch), lstride,
                       float(scale), out, out16=out16, ws=ws)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    ref = O.attn_decode_f16(q, k, v, kb, ke, scale)
    rel = np.abs(got - ref).max() / np.abs(ref).max()
    assert rel <= 2e-3, rel
    assert rel <= 1e-5, rel
    # the fp16 output is the fp32 output rounded to nearest even
    assert np.array_equal(out16.cpu().numpy(), got.astype(np.float16))


@pytest.mark.parametrize("B,lstride", [(16, 1000), (3, 300), (40, 200), (64, 700), (1, 64)])
def test_qkv_attn_fused_equals_separate_kernels(gpu, B, lstride):
    """The decode path's fused QKV + attention kernel equals the LN-input QKV GEMV, the fp16 K/V
    append and the standalone decode attention, to the bit (output, Q8_0 copy, cache, LN row)."""
    import torch
    rng = np.random.default_rng(4000 + B)
    D, nh = 512, 16
    n = 3 * D
    W = rng.standard_normal((n, D)).astype(np.float32) * 0.02
    wbk = sm.q8_quantize_ref(W).ravel()
    wq = torch.zeros(n * D, dtype=torch.int8, device="cuda")
    wd = torch.zeros(n * D // 32, dtype=torch.int16, device="cuda")
    gpu.op_q8_repack(_dev(wbk, torch), n, D, wq, wd)
    bias = _dev(rng.standard_normal(n).astype(np.float32) * 0.02, torch)
    res = _dev(rng.standard_normal((B, D)).astype(np.float32), torch)
    r = _dev(rng.standard_normal((B, D)).astype(np.float32) * 0.5, torch)
    lb = _dev(rng.standard_normal(D).astype(np.float32) * 0.02, torch)
    wb = _dev(np.concatenate([1 + 0.05 * rng.standard_normal(D), 0.05 * rng.standard_normal(D)]).astype(np.float32),
              torch)
    kc = _dev(rng.standard_normal((B, nh, lstride, 32)).astype(np.float16), torch)
    vc = _dev(rng.standard_normal((B, nh, lstride, 32)).astype(np.float16), torch)
    col = lstride - 3
    begins = rng.integers(0, col + 1, B).astype(np.int32)
    begins[0] = 0
    if B > 2:
        begins[1] = col                     # only the new key is valid
    kb = _dev(begins, torch)
    col_d = torch.tensor([col], dtype=torch.int32, device="cuda")
    scale = float(1.0 / np.sqrt(32.0))
    # fused
    k1, v1 = kc.clone(), vc.clone()
    out1 = torch.zeros((B, D), dtype=torch.float32, device="cuda")
    oq1 = torch.zeros(B * D, dtype=torch.int8, device="cuda")
    od1 = torch.zeros(B * nh, dtype=torch.float32, device="cuda")
    ln1 = torch.zeros((B, D), dtype=torch.float32, device="cuda")
    gpu.op_qkv_attn(wq, wd, bias, res, r, lb, wb, k1, v1, kb, col_d, scale, out1, oq=oq1, od=od1, ln_out=ln1)
    # separate kernels
    k2, v2 = kc.clone(), vc.clone()
    qkv = torch.zeros((B, n), dtype=torch.float32, device="cuda")
    ln2 = torch.zeros((B, D), dtype=torch.float32, device="cuda")
    gpu.op_ln_gemv(wq, wd, n, res, r, lb, wb, bias, 0, qkv, ln_out=ln2)
    k2[:, :, col, :] = qkv[:, D:2 * D].reshape(B, nh, 32).half()
    v2[:, :, col, :] = qkv[:, 2 * D:].reshape(B, nh, 32).half()
    out2 = torch.zeros((B, D), dtype=torch.float32, device="cuda")
    oq2 = torch.zeros(B * D, dtype=torch.int8, device="cuda")
    od2 = torch.zeros(B * nh, dtype=torch.float32, device="cuda")
    ws = torch.zeros(gpu.attn_workspace_bytes(B, nh, lstride), dtype=torch.uint8, device="cuda")
    ke = torch.full((B,), col + 1, dtype=torch.int32, device="cuda")
    gpu.op_attn_decode(qkv[:, :D].reshape(B, nh, 32).contiguous(), k2.view(torch.int16), v2.view(torch.int16), kb,
                       ke, lstride, scale, out2, oq=oq2, od=od2, ws=ws)
    torch.cuda.synchronize()
    assert torch.equal(ln1, ln2)
    assert torch.equal(k1, k2) and torch.equal(v1, v2)
    assert torch.equal(out1, out2), (out1 - out2).abs().max().item()
    assert torch.equal(oq1, oq2) and torch.equal(od1, od2)


@pytest.mark.parametrize("n,k", [(1536, 512), (512, 512), (2048, 512), (512, 2048)])
@pytest.mark.parametrize("m", [1, 16, 100, 300, 1024])
def test_q8_gemm_matches_oracle(gpu, n, k, m):
    """The MFMA GEMM computes the same Q8_0 products as ggml-cpu's mul_mat; only the fp32
    accumulation order differs (per block instead of 8 lanes + hsum): within 2e-6 of the output
    scale, i.e. a few fp32 ulps. Its operands carry the quants in natural order."""
    import torch
    rng = np.random.default_rng(7000 + n + k + m)
    W = rng.standard_normal((n, k)).astype(np.float32) * 0.02
    X = rng.standard_normal((m, k)).astype(np.float32)
    X[0, :64] = 0.0
    wb = sm.q8_quantize_ref(W).ravel()
    wq_n, wd_n = blocks_to_split(wb, n, k)                  # natural-order quants, fp16 scales
    xq_n, xd_n = blocks_to_split(O.q8_quantize_x86(X), m, k)
    wq = _dev(wq_n, torch)
    wd = _dev(wd_n.view(np.int16), torch)
    xq = _dev(xq_n, torch)
    xd = _dev(xd_n.view(np.float16).astype(np.float32), torch)
    bias = rng.standard_normal(n).astype(np.float32) * 0.02
    y = torch.zeros((m, n), dtype=torch.float32, device="cuda")
    gpu.op_q8_gemm(wq, wd, n, k, xq, xd, m, None, 0, y)
    y2 = torch.zeros((m, n), dtype=torch.float32, device="cuda")
    gpu.op_q8_gemm(wq, wd, n, k, xq, xd, m, _dev(bias, torch), 1, y2)
    torch.cuda.synchronize()
    ref = O.q8_matmul(wb, n, k, X)
    got = y.cpu().numpy()
    scale = np.abs(ref).max()
    assert np.abs(got - ref).max() <= 2e-6 * scale, np.abs(got - ref).max() / scale
    ref2 = np.maximum(ref + bias[None, :], 0.0)
    assert np.abs(y2.cpu().numpy() - ref2).max() <= 2e-6 * scale


@pytest.mark.parametrize("n,k", [(2048, 512), (512, 2048), (1024, 4096)])
@pytest.mark.parametrize("m", [300, 1024])
@pytest.mark.parametrize("with_y", [True, False])
def test_q8_gemm_large_q8_out(gpu, n, k, m, with_y):
    """The 128 x 128 GEMM (above 256 rows) with bias + ReLU: the fp32 rows within 2e-6 of the
    oracle's scale, the Q8_0 rows the x86 quantisation of those fp32 rows bit for bit, rows past m
    untouched. Two epilogues: fp32 + Q8_0 (a block is 8 lanes of 4 columns) and Q8_0 alone (a
    block is 2 lanes of 16 columns; its fp32 rows then come from a second call with fp32 only)."""
    import torch
    rng = np.random.default_rng(7200 + n + k + m)
    W = rng.standard_normal((n, k)).astype(np.float32) * 0.02
    X = rng.standard_normal((m, k)).astype(np.float32)
    X[1, :] = 0.0                       # an all-zero row: zero blocks (scale 0) in the output
    wb = sm.q8_quantize_ref(W).ravel()
    wq_n, wd_n = blocks_to_split(wb, n, k)
    xq_n, xd_n = blocks_to_split(O.q8_quantize_x86(X), m, k)
    wq, wd = _dev(wq_n, torch), _dev(wd_n.view(np.int16), torch)
    xq, xd = _dev(xq_n, torch), _dev(xd_n.view(np.float16).astype(np.float32), torch)
    b = rng.standard_normal(n).astype(np.float32) * 0.02
    b[:32] = 0.0                        # with row 1 at zero: a block of exact zeros
    bias = _dev(b, torch)
    y = torch.full((m + 1, n), 7.0, dtype=torch.float32, device="cuda")
    yq = torch.full((m + 1, n), 5, dtype=torch.int8, device="cuda")
    yd = torch.full((m + 1, n // 32), 3.0, dtype=torch.float32, device="cuda")
    if with_y:
        gpu.op_q8_gemm_ex(wq, wd, n, k, xq, xd, m, bias, 1, y, yq, yd)
    else:
        gpu.op_q8_gemm_ex(wq, wd, n, k, xq, xd, m, bias, 1, None, yq, yd)
        gpu.op_q8_gemm_ex(wq, wd, n, k, xq, xd, m, bias, 1, y, None, None)
    torch.cuda.synchronize()
    y, yq, yd = y.cpu().numpy(), yq.cpu().numpy(), yd.cpu().numpy()
    assert (y[m] == 7.0).all() and (yq[m] == 5).all() and (yd[m] == 3.0).all()
    y, yq, yd = y[:m], yq[:m], yd[:m]
    ref = np.maximum(O.q8_matmul(wb, n, k, X) + b[None, :], 0.0)
    assert np.abs(y - ref).max() <= 2e-6 * np.abs(ref).max()
    assert (yd[1, 0] == 0.0) and (yq[1, :32] == 0).all()
    q_ref, d_ref = blocks_to_split(O.q8_quantize_x86(y), m, n)
    assert np.array_equal(yq, q_ref.reshape(m, n))
    assert np.array_equal(yd, d_ref.view(np.float16).astype(np.float32).reshape(m, n // 32))


@pytest.mark.parametrize("n,k", [(1536, 512), (2048, 512), (512, 2048)])
@pytest.mark.parametrize("m", [300, 1000])
def test_q8h_gemm_fp16_mode(gpu, n, k, m):
    """The projection of the prefill's fp16 mode: the weights dequantised to fp16(d * q) bit for
    bit (numpy's float16 conversion rounds to nearest even); the GEMM is the fp32-accumulated
    product of the activations fp16(dx * qx) and those weights (within 2e-5 of the row's scale of
    a float64 product of the same fp16 operands), and within 2e-3 of the row's scale of ggml's
    Q8_0 product (the oracle), with bias + ReLU; rows past m untouched; its Q8_0 output is the x86
    quantisation of its own fp32 output."""
    import torch
    rng = np.random.default_rng(7300 + n + k + m)
    W = rng.standard_normal((n, k)).astype(np.float32) * 0.02
    X = rng.standard_normal((m, k)).astype(np.float32)
    X[1, :] = 0.0
    wb = sm.q8_quantize_ref(W).ravel()
    wq_n, wd_n = blocks_to_split(wb, n, k)
    xq_n, xd_n = blocks_to_split(O.q8_quantize_x86(X), m, k)
    wq, wd = _dev(wq_n, torch), _dev(wd_n.view(np.int16), torch)
    xq, xd = _dev(xq_n, torch), _dev(xd_n.view(np.float16).astype(np.float32), torch)
    b = rng.standard_normal(n).astype(np.float32) * 0.02
    bias = _dev(b, torch)
    w16 = torch.zeros(n * k, dtype=torch.int16, device="cuda")
    gpu.op_q8_dequant_f16(wq, wd, n, k, w16)

    def deq(q, d, rows):
        return (q.reshape(rows, k // 32, 32).astype(np.float32) *
                d.view(np.float16).astype(np.float32).reshape(rows, k // 32, 1)).astype(np.float16).reshape(rows, k)

    w16_ref = deq(wq_n, wd_n, n)
    torch.cuda.synchronize()
    assert np.array_equal(w16.cpu().numpy().reshape(n, k), w16_ref.view(np.int16))
    y = torch.full((m + 1, n), 7.0, dtype=torch.float32, device="cuda")
    yq = torch.full((m + 1, n), 5, dtype=torch.int8, device="cuda")
    yd = torch.full((m + 1, n // 32), 3.0, dtype=torch.float32, device="cuda")
    gpu.op_q8h_gemm(w16, n, k, xq, xd, m, bias, 1, y=y)
    gpu.op_q8h_gemm(w16, n, k, xq, xd, m, bias, 1, yq=yq, yd=yd)
    torch.cuda.synchronize()
    y, yq, yd = y.cpu().numpy(), yq.cpu().numpy(), yd.cpu().numpy()
    assert (y[m] == 7.0).all() and (yq[m] == 5).all() and (yd[m] == 3.0).all()
    y, yq, yd = y[:m], yq[:m], yd[:m]
    ref16 = np.maximum(deq(xq_n, xd_n, m).astype(np.float64) @ w16_ref.astype(np.float64).T + b[None, :], 0.0)
    ref = np.maximum(O.q8_matmul(wb, n, k, X) + b[None, :], 0.0)
    scale = np.maximum(np.abs(ref).max(axis=1), 1e-6)
    err16 = (np.abs(y - ref16).max(axis=1) / scale).max()
    err = (np.abs(y - ref).max(axis=1) / scale).max()
    print(f"fp16 GEMM n={n} k={k} m={m}: vs the same fp16 operands {err16:.2e}, vs ggml's Q8_0 product {err:.2e}")
    assert err16 <= 2e-5 and err <= 2e-3
    q_ref, d_ref = blocks_to_split(O.q8_quantize_x86(y), m, n)
    assert np.array_equal(yq, q_ref.reshape(m, n))
    assert np.array_equal(yd, d_ref.view(np.float16).astype(np.float32).reshape(m, n // 32))


@pytest.mark.parametrize("n,k", [(1536, 512), (512, 2048), (2048, 512)])
@pytest.mark.parametrize("m", [1, 64, 100, 128, 256])
def test_q8_gemm_small_tiles(gpu, n, k, m):
    """The small-batch GEMM (32-column tiles, K split over 4 waves): every row tiling (1, 2, 4
    tiles of 32 rows per workgroup) gives the same bits, within 2e-6 of the oracle's scale; with
    bias + ReLU its Q8_0 output is the x86 quantisation of its own fp32 output (natural order)."""
    import torch
    rng = np.random.default_rng(7100 + n + k + m)
    W = rng.standard_normal((n, k)).astype(np.float32) * 0.02
    X = rng.standard_normal((m, k)).astype(np.float32)
    wb = sm.q8_quantize_ref(W).ravel()
    wq_n, wd_n = blocks_to_split(wb, n, k)
    xq_n, xd_n = blocks_to_split(O.q8_quantize_x86(X), m, k)
    wq, wd = _dev(wq_n, torch), _dev(wd_n.view(np.int16), torch)
    xq, xd = _dev(xq_n, torch), _dev(xd_n.view(np.float16).astype(np.float32), torch)
    bias = _dev(rng.standard_normal(n).astype(np.float32) * 0.02, torch)
    ref = O.q8_matmul(wb, n, k, X)
    scale = np.abs(ref).max()
    outs = []
    for tr in (1, 2, 4):
        y = torch.zeros((m, n), dtype=torch.float32, device="cuda")
        yq = torch.zeros((m, n), dtype=torch.int8, device="cuda")
        yd = torch.zeros((m, n // 32), dtype=torch.float32, device="cuda")
        gpu.op_q8_gemm_ex(wq, wd, n, k, xq, xd, m, bias, 1, y, yq, yd, tile_rows=tr)
        torch.cuda.synchronize()
        outs.append((y.cpu().numpy(), yq.cpu().numpy(), yd.cpu().numpy()))
    for y, yq, yd in outs[1:]:
        assert np.array_equal(y, outs[0][0]) and np.array_equal(yq, outs[0][1]) and np.array_equal(yd, outs[0][2])
    y, yq, yd = outs[0]
    ref_relu = np.maximum(ref + bias.cpu().numpy()[None, :], 0.0)
    assert np.abs(y - ref_relu).max() <= 2e-6 * scale
    q_ref, d_ref = blocks_to_split(O.q8_quantize_x86(y), m, n)
    assert np.array_equal(yq, q_ref.reshape(m, n))
    assert np.array_equal(yd, d_ref.view(np.float16).astype(np.float32).reshape(m, n // 32))
    # the same product on operands in the matrix-core order (whole-line loads): the same bits, and
    # the Q8_0 output in that order
    wq_t, wd_t = to_tiled(wq_n, wd_n.view(np.int16))
    xq_t, xd_t = to_tiled(xq_n, xd_n.view(np.float16).astype(np.float32))
    mp = (m + 31) // 32 * 32
    yt = torch.zeros((m, n), dtype=torch.float32, device="cuda")
    yqt = torch.zeros(mp * n, dtype=torch.int8, device="cuda")
    ydt = torch.zeros(mp * n // 32, dtype=torch.float32, device="cuda")
    gpu.op_q8_gemm_ex(_dev(wq_t, torch), _dev(wd_t, torch), n, k, _dev(xq_t, torch), _dev(xd_t, torch), m, bias, 1,
                      yt, yqt, ydt, tiled=True)
    torch.cuda.synchronize()
    assert np.array_equal(yt.cpu().numpy(), y)
    qt_ref, dt_ref = to_tiled(yq, yd)
    assert np.array_equal(yqt.cpu().numpy(), qt_ref) and np.array_equal(ydt.cpu().numpy(), dt_ref)


@pytest.mark.parametrize("B,S,max_len,pads,what", [
    (3, 300, 100, [0, 17, 60], "text + causal semantic rows, left pads, ragged last tile"),
    (1, 64, 64, [5], "text rows only"),
    (2, 130, 1, [0, 0], "one text row; every other row causal"),
    (2, 33, 20, [19, 3], "a one-key text span; 33 rows"),
    (2, 1024, 300, [0, 123], "long prompt (1024 rows of which 724 semantic)"),
])
@pytest.mark.parametrize("path", [1, 2, 3])
def test_attn_prefill_matches_oracle(gpu, B, S, max_len, pads, what, path):
    """Both prefill-attention kernels (1: lane per query, 2: matrix cores with fp16 hi + lo
    operands; 3: the same with the weighted sum of fp16 probabilities and values, the prefill's
    fp16 mode) against the oracle; the Q8_0 copy is the x86 quantisation of the fp32 output."""
    import torch
    nh, D = 16, 512
    rng = np.random.default_rng(40 + S + path)
    qkv = rng.standard_normal((B, S, 3 * D)).astype(np.float32)
    qkv[:, :, :D] *= 2.0            # sharper softmax than unit scores
    pad = np.array(pads, np.int32)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(32)))
    out = torch.zeros(B * S * D, dtype=torch.float32, device="cuda")
    oq = torch.zeros(B * S * D, dtype=torch.int8, device="cuda")
    od = torch.zeros(B * S * D // 32, dtype=torch.float32, device="cuda")
    gpu.op_attn_prefill(_dev(qkv, torch), max_len, _dev(pad, torch), nh, scale, out, oq, od, path=path)
    torch.cuda.synchronize()
    got = out.cpu().numpy().reshape(B, S, D)
    ref = O.attn_prefill(qkv, max_len, pad, nh, scale)
    rel = np.abs(got - ref).max() / np.abs(ref).max()
    print(f"attention path {path}, {what}: {rel:.2e} of the output's scale")
    assert rel <= 2e-3, rel
    if path != 3:
        assert rel <= 2e-5, rel   # fp32 (or hi + lo split) products with fp32 accumulation
    q_ref, d_ref = blocks_to_split(O.q8_quantize_x86(got.reshape(B * S, D)), B * S, D)
    q_got = oq.cpu().numpy()
    # quants in the layout of the projection that reads them: sliced (GEMV) or natural (GEMM)
    q_got = unslice(q_got, D) if path == 1 else q_got.reshape(B * S, D)
    assert np.array_equal(q_got, q_ref)
    d_ref32 = d_ref.view(np.float16).astype(np.float32)
    assert np.array_equal(od.cpu().numpy().reshape(B * S, -1).view(np.uint32), d_ref32.view(np.uint32))


def test_attn_prefill_decoder_dispatch(gpu):
    """Path 4, the matrix-core prefill attention as the decoder's prefill dispatches it (sequences
    longest first, query blocks last first, waves of 32 padding queries skipped), with left pads
    that do not fall on a 32-query wave or a 256-query workgroup boundary: every row of a valid
    query and every padding row that shares a wave with one equals path 2's to the bit (and the
    oracle within 2e-5); the rows of padding-only waves are zero."""
    import torch
    nh, D = 16, 512
    B, S, max_len = 5, 384, 320
    pads = np.array([0, 17, 33, 255, 300], np.int32)
    rng = np.random.default_rng(77)
    qkv = rng.standard_normal((B, S, 3 * D)).astype(np.float32)
    qkv[:, :, :D] *= 2.0
    scale = float(np.float32(1.0) / np.sqrt(np.float32(32)))
    outs = {}
    for path in (2, 4):
        out = torch.zeros(B * S * D, dtype=torch.float32, device="cuda")
        oq = torch.zeros(B * S * D, dtype=torch.int8, device="cuda")
        od = torch.zeros(B * S * D // 32, dtype=torch.float32, device="cuda")
        gpu.op_attn_prefill(_dev(qkv, torch), max_len, _dev(pads, torch), nh, scale, out, oq, od, path=path)
        torch.cuda.synchronize()
        outs[path] = (out.cpu().numpy().reshape(B, S, D), oq.cpu().numpy().reshape(B, S, D),
                      od.cpu().numpy().reshape(B, S, D // 32))
    ref = O.attn_prefill(qkv, max_len, pads, nh, scale)
    a, b4 = outs[2], outs[4]
    n_zero = 0
    for b in range(B):
        for s in range(S):
            if (s // 32) * 32 + 32 <= pads[b]:          # a wave of padding queries only
                assert np.all(b4[0][b, s] == 0.0), (b, s)
                n_zero += 1
            else:
                assert np.array_equal(b4[0][b, s].view(np.uint32), a[0][b, s].view(np.uint32)), (b, s)
                assert np.array_equal(b4[1][b, s], a[1][b, s]) and np.array_equal(b4[2][b, s], a[2][b, s]), (b, s)
    assert n_zero == sum(int(p) // 32 * 32 for p in pads)
    valid = np.concatenate([ref[b, pads[b]:] - b4[0][b, pads[b]:] for b in range(B)])
    assert np.abs(valid).max() / np.abs(ref).max() <= 2e-5

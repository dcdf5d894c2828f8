"""GPU parity of the trait Backend operators against the CPU oracle.

Inputs are identical seeded arrays on both sides.  Bar (per kernel, f32):
|gpu - oracle| <= 1e-4 + 1e-3 * |oracle|; the GEMV's integer block sums are
exact, only the f32 order of the block accumulation differs.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import rel_close

pytestmark = pytest.mark.gpu
F32 = np.float32

# (n, k): every decode GEMV shape of the 1B, 8B and 70B workloads (q, k|v,
# o, gate|up, down, lm_head) plus the reference's own test shapes.
GEMV_SHAPES = [
    (64, 128), (128, 256), (2048, 2048), (512, 2048), (16384, 2048), (2048, 8192),
    (128256, 2048), (4096, 4096), (1024, 4096), (28672, 4096), (4096, 14336), (128256, 4096),
    (8192, 8192), (1024, 8192), (57344, 8192), (8192, 28672), (128256, 8192),
]


def _x(rng, m, k):
    return rng.normal(0, 1, (m, k)).astype(F32)


@pytest.mark.parametrize("n,k", GEMV_SHAPES)
def test_gemv_q4_0(hip, orc, rng, n, k):
    be = hip.HipBackend()
    qs, sc = hip.synth_q4(20260002, n * 7 + k, n, k, 0.003, 0.006)
    x = _x(rng, 1, k)
    w = hip.Tensor.from_q4(qs, sc, n, k)
    assert w.dtype == hip.DType.Q4_0
    got = be.matmul_transposed(hip.Tensor.from_numpy(x), w).data()
    want = orc.matmul_transposed_q4(x, qs, sc, n)
    ok, err, nbad = rel_close(got, want)
    assert ok, f"max err {err}, {nbad} outside tolerance"


@pytest.mark.parametrize("m,n,k", [(1, 64, 128), (4, 128, 256), (3, 4096, 4096)])
def test_gemv_q4_reference_quantiser_rows(hip, orc, rng, m, n, k):
    """Weights from the reference quantiser (f32 scales, Storage::CpuQ4) and
    M>1 rows (test_opencl_q4_prefill_stress, test/opencl.rs:475-510)."""
    be = hip.HipBackend()
    b = rng.uniform(-1, 1, (n, k)).astype(F32)
    qs, sc = orc.quantize_q4(b)
    w = hip.Tensor.from_q4(qs, sc, n, k)
    assert w.dtype == hip.DType.Q4
    a = rng.uniform(-1, 1, (m, k)).astype(F32)
    got = be.matmul_transposed(hip.Tensor.from_numpy(a), w).data()
    want = orc.matmul_transposed_q4(a, qs, sc, n)
    ok, err, nbad = rel_close(got, want)
    assert ok, f"max err {err}, {nbad} outside tolerance"


@pytest.mark.parametrize("n,k", [(64, 128), (2048, 2048), (512, 2048), (16384, 2048), (2048, 8192)])
def test_gemv_q8_0(hip, orc, rng, n, k):
    be = hip.HipBackend()
    qs, sc = hip.synth_q8(20260001, n + k, n, k, 2e-4, 3.5e-4)
    x = _x(rng, 1, k)
    w = hip.Tensor.from_q8_0(qs, sc, n, k)
    got = be.matmul_transposed(hip.Tensor.from_numpy(x), w).data()
    want = orc.matmul_transposed_q8w(x, qs, sc, n)
    ok, err, nbad = rel_close(got, want)
    assert ok, f"max err {err}, {nbad} outside tolerance"


# (m, n, k): prompt-batch GEMMs.  m and n cover full and ragged 128-row
# tiles; k covers one block, a partial and several 16-block scale chunks.
GEMM_SHAPES = [(2, 64, 32), (37, 256, 4096), (200, 1000, 1024), (130, 4096, 256),
               (129, 6144, 4096), (512, 128, 14336)]


@pytest.mark.parametrize("wtype", ["q4_0", "q4_ref", "q8_0"])
@pytest.mark.parametrize("m,n,k", GEMM_SHAPES)
def test_gemm_bit_exact(hip, orc, rng, wtype, m, n, k):
    """M > 1 rows (cpu.rs:90-110): per-row Q8_0 codes, then per output the
    block loop total += isum_b * (d_w * d_a) from 0.0 in block order.  The
    int8 MFMA gives every isum_b exactly and the epilogue keeps the order, so
    the GPU result equals the oracle bit for bit."""
    be = hip.HipBackend()
    a = _x(rng, m, k)
    a[0, :32] = 0.0                  # an all-zero block (d_a = 0)
    a[m - 1, 5] = 1e-30              # a tiny value next to the block maximum
    if wtype == "q8_0":
        qs, sc = hip.synth_q8(20260003, m + n + k, n, k, 2e-4, 3.5e-4)
        w = hip.Tensor.from_q8_0(qs, sc, n, k)
        want = orc.matmul_transposed_q8w(a, qs, sc, n)
    else:
        if wtype == "q4_0":
            qs, sc = hip.synth_q4(20260004, m + n + k, n, k, 0.003, 0.006)
        else:
            qs, sc = orc.quantize_q4(rng.uniform(-1, 1, (n, k)).astype(F32))
        w = hip.Tensor.from_q4(qs, sc, n, k)
        want = orc.matmul_transposed_q4(a, qs, sc, n)
    got = be.matmul_transposed(hip.Tensor.from_numpy(a), w).data()
    bad = np.nonzero(got != want)
    assert bad[0].size == 0, (
        f"{bad[0].size} of {got.size} outputs differ; first at {bad[0][0]},{bad[1][0]}: "
        f"{got[bad[0][0], bad[1][0]]!r} vs {want[bad[0][0], bad[1][0]]!r}")


@pytest.mark.parametrize("k", [256, 4096])
def test_gemv_zero_and_special_inputs(hip, orc, k):
    """amax == 0 blocks (d = 0), a NaN input element (code 0) and, at
    k = 4096 (eight lanes per block in the prologue), a block whose amax is
    subnormal (d = amax/127 subnormal, 1/d = inf, codes clamp to +-127)."""
    be = hip.HipBackend()
    n = 96
    qs, sc = hip.synth_q4(3, 4, n, k, 0.003, 0.006)
    x = np.zeros((1, k), F32)
    x[0, 40:70] = np.linspace(-2, 2, 30)
    x[0, 200] = np.nan
    if k > 1024:
        x[0, 1000:1032] = np.linspace(-1e-40, 1e-40, 32, dtype=F32)
        x[0, 3000:3064] = np.linspace(-5, 3, 64)
    w = hip.Tensor.from_q4(qs, sc, n, k)
    got = be.matmul_transposed(hip.Tensor.from_numpy(x), w).data()
    want = orc.matmul_transposed_q4(x, qs, sc, n)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok, err, _ = rel_close(np.nan_to_num(got), np.nan_to_num(want))
    assert ok, err


def test_matmul_f32_bit_exact(hip, orc, rng):
    be = hip.HipBackend()
    for (m, k, n) in [(1, 128, 256), (16, 64, 32)]:
        a = rng.uniform(-1, 1, (m, k)).astype(F32)
        a[0, 3] = 0.0
        b = rng.uniform(-1, 1, (k, n)).astype(F32)
        got = be.matmul(hip.Tensor.from_numpy(a), hip.Tensor.from_numpy(b)).data()
        assert np.array_equal(got, orc.matmul(a, b))


def test_matmul_transposed_f32_and_slice_bit_exact(hip, orc, rng):
    be = hip.HipBackend()
    a = rng.uniform(-1, 1, (4, 128)).astype(F32)
    b = rng.uniform(-1, 1, (64, 128)).astype(F32)
    got = be.matmul_transposed(hip.Tensor.from_numpy(a), hip.Tensor.from_numpy(b)).data()
    assert np.array_equal(got, orc.matmul_transposed_f32(a, b))
    q = rng.uniform(-1, 1, (1, 64)).astype(F32)
    kc = rng.uniform(-1, 1, (10, 64)).astype(F32)
    got = be.matmul_slice(hip.Tensor.from_numpy(q), kc, 10, 64).data()
    assert np.array_equal(got, orc.matmul_slice(q, kc, 10))


def test_rms_norm(hip, orc, rng):
    be = hip.HipBackend()
    d = be.rms_norm(hip.Tensor.from_numpy(np.array([[1, 2, 3, 4]], F32)),
                    hip.Tensor.from_numpy(np.ones(4, F32)), 1e-5).data()[0]
    assert abs(d[0] - 0.3651) < 1e-3 and abs(d[3] - 1.4605) < 1e-3
    # the sum of squares is folded in index order as the reference does
    # (cpu.rs:381): bit-exact, also for rows longer than one staging chunk
    for dim in (4096, 5000):
        x = rng.normal(0, 1, (7, dim)).astype(F32)
        w = rng.normal(1, 0.02, dim).astype(F32)
        got = be.rms_norm(hip.Tensor.from_numpy(x), hip.Tensor.from_numpy(w), 1e-5).data()
        assert np.array_equal(got, orc.rms_norm(x, w, 1e-5)), dim


def test_softmax(hip, orc, rng):
    be = hip.HipBackend()
    d = be.softmax(hip.Tensor.from_numpy(np.array([[1, 2, 3]], F32))).data()[0]
    assert abs(d.sum() - 1) < 1e-5 and d[2] > d[1] > d[0]
    # glibc's expf and the sum in index order (cpu.rs:410-415): bit-exact
    x = rng.normal(0, 3, (5, 3000)).astype(F32)
    x[1, 500:] = -np.inf  # causal-mask style row
    x[2, :] = 0.0         # a flat row
    x[3, 7] = 120.0       # one dominant entry: the others underflow
    got = be.softmax(hip.Tensor.from_numpy(x)).data()
    assert np.array_equal(got, orc.softmax(x))


def test_rope_bit_exact(hip, orc, rng):
    be = hip.HipBackend()
    t = hip.Tensor.from_numpy(np.array([[1, 0, 0, 1]], F32))
    be.rope_inplace(t, 1)
    d = t.data()[0]
    assert abs(np.hypot(d[0], d[2]) - 1) < 1e-4 and d[0] != 1.0
    for hd, pos in [(64, 0), (64, 31), (128, 511), (128, 8190)]:
        x = rng.normal(0, 1, (3, hd)).astype(F32)
        t = hip.Tensor.from_numpy(x)
        be.rope_inplace(t, pos)
        assert np.array_equal(t.data(), orc.rope_inplace(x, pos))


def test_mixed_f16_product_equals_convert_multiply(hip):
    """The reference-order attention multiplies f32 by f16 cache values with
    one mixed-precision FMA (addend -0) instead of a conversion and a
    multiply; its results must be the same bits for every f16 pattern.  The
    f32 side: signed zeros, denormals, the normal range ends, infinities, a
    NaN, powers of two, and random bit patterns and attention-sized values."""
    special = np.array([0x00000000, 0x80000000, 0x00000001, 0x80000001, 0x007FFFFF, 0x00800000,
                        0x7F7FFFFF, 0xFF7FFFFF, 0x7F800000, 0xFF800000, 0x7FC00000, 0x3F800000,
                        0xBF800000, 0x00400000, 0x0F800000, 0x1F800000, 0x33800000, 0x7E800000,
                        0x477FE000, 0x38800000, 0x33000000], dtype=np.uint32).view(F32)
    g = np.random.default_rng(12345)
    bits = g.integers(0, 2**32, 2048, dtype=np.uint64).astype(np.uint32).view(F32)
    vals = np.concatenate([special, bits, g.uniform(-20, 20, 2048).astype(F32),
                           g.uniform(0, 1, 1024).astype(F32)])
    bad = hip.HipBackend().check_mul_f16(hip.Tensor.from_numpy(vals)).data()
    assert bad.shape == (65536,)
    assert int(bad.sum()) == 0, f"{int(np.count_nonzero(bad))} f16 patterns differ, e.g. {np.nonzero(bad)[0][:8]}"


def test_elementwise(hip, orc, rng):
    be = hip.HipBackend()
    a = rng.uniform(-1, 1, (10, 10)).astype(F32)
    b = rng.uniform(-1, 1, (10, 10)).astype(F32)
    ta = hip.Tensor.from_numpy(a)
    be.add_assign(ta, hip.Tensor.from_numpy(b))
    assert np.array_equal(ta.data(), orc.add_assign(a, b))
    # SiLU with glibc's expf (layer.rs:75-79): bit-exact over a wide range,
    # including the exp overflow and underflow ends
    g = np.concatenate([rng.uniform(-1, 1, 4096), rng.normal(0, 30, 4096),
                        [-200.0, -88.8, -88.7, 0.0, 87.0, 104.0, 200.0]]).astype(F32)
    u = rng.uniform(-1, 1, g.size).astype(F32)
    tg = hip.Tensor.from_numpy(g)
    be.silu_mul(tg, hip.Tensor.from_numpy(u))
    assert np.array_equal(tg.data(), orc.silu_mul(g, u))
    s = be.scale(hip.Tensor.from_numpy(a), 0.088388).data()
    assert np.array_equal(s, orc.scale(a, 0.088388))
    c = be.copy_from(hip.Tensor.from_numpy(a)).data()
    assert np.array_equal(c, a)


def test_memory_sync_loop(hip):
    """test_opencl_memory_sync_loop (test/opencl.rs:413-437): 100 add_assign."""
    be = hip.HipBackend()
    acc = hip.Tensor.zeros((1024,))
    one = hip.Tensor.from_numpy(np.ones(1024, F32))
    for _ in range(100):
        be.add_assign(acc, one)
    assert np.all(acc.data() == 100.0)


def test_shape_errors(hip):
    be = hip.HipBackend()
    a = hip.Tensor.from_numpy(np.ones((2, 64), F32))
    b = hip.Tensor.from_numpy(np.ones((3, 32), F32))
    with pytest.raises(hip.LlmrsError) as e:
        be.matmul_transposed(a, b)
    assert e.value.code == hip.E_INVALID
    with pytest.raises(hip.LlmrsError):
        be.add_assign(a, b)

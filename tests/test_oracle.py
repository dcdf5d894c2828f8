"""Pins the CPU oracle (oracle/oracle.cpp) before the tests trust it as their reference.

Each reference known-answer test (src/test/cpu.rs, src/test/opencl.rs,
src/core/layer.rs tests) is restated, and every function is also checked
against an independent closed form or brute force (tests/numpy_ref.py) chosen
so that a dropped term, a wrong sign/index or a transposed operand fails.
"""
from __future__ import annotations

import numpy as np
import pytest

import numpy_ref as ref

F32 = np.float32


# ---- quantize_row_q8_0 (cpu.rs:724-743) ------------------------------------
def test_q8_quantize_closed_form(orc, rng):
    x = rng.uniform(-3, 3, 32 * 64).astype(F32)
    q, d = orc.quantize_row_q8_0(x)
    q2, d2 = ref.q8_quantize(x)
    assert np.array_equal(d, d2)
    assert np.array_equal(q, q2)


def test_q8_quantize_edges(orc):
    x = np.zeros(96, F32)
    # block 0: amax = 0 -> d = 0, all codes 0 (cpu.rs:732-734)
    # block 1: amax = 127 -> d = 1, inv = 1: ties round away from zero
    x[32:64] = [127.0, 2.5, -2.5, 0.5, -0.5, 1.5, -1.5] + [0.0] * 25
    # block 2: the amax element maps to +-127 exactly
    x[64] = -5.0
    x[65] = 2.5
    q, d = orc.quantize_row_q8_0(x)
    assert d[0] == 0.0 and not q[:32].any()
    assert d[1] == 1.0
    assert list(q[32:39]) == [127, 3, -3, 1, -1, 2, -2]
    assert q[64] == -127
    assert d[2] == F32(F32(5.0) / F32(127.0))


def test_q8_quantize_nan_is_zero(orc):
    x = np.ones(32, F32)
    x[3] = np.nan
    q, d = orc.quantize_row_q8_0(x)
    assert q[3] == 0 and d[0] == F32(1.0) / F32(127.0) and q[0] == 127


# ---- Q4 format (tensor.rs:102-167, test/opencl.rs:182-235) -----------------
def test_round_half_away_identity():
    """The GPU quantiser rounds with trunc(p + copysign(0.5 - 2**-25, p))
    instead of roundf (fewer instructions).  Pin that this equals Rust's
    f32::round (half away from zero, cpu.rs:739) on every float32 within
    +-64 ulps of each integer and half-integer up to 256 (where a wrong
    constant or a double rounding would show), plus random values; an
    exhaustive check over all 2**32 bit patterns also finds no difference."""
    F32 = np.float32
    centers = np.concatenate([np.arange(0, 257, dtype=np.float64), np.arange(0, 256, dtype=np.float64) + 0.5])
    vals = []
    for c in centers:
        x = F32(c)
        seq_up = [x]
        seq_dn = [x]
        u, d = x, x
        for _ in range(64):
            u = np.nextafter(u, F32(np.inf))
            d = np.nextafter(d, F32(-np.inf))
            seq_up.append(u)
            seq_dn.append(d)
        vals.extend(seq_up)
        vals.extend(seq_dn)
    rng = np.random.default_rng(5)
    x = np.concatenate([np.array(vals, F32), rng.uniform(-300, 300, 1 << 20).astype(F32),
                        rng.uniform(-2, 2, 1 << 20).astype(F32),
                        np.array([0.0, -0.0, 0.49999997, -0.49999997, 0.5, -0.5, 1.5, 2.5, 126.5, 127.5,
                                  np.inf, -np.inf, 1e-40, -1e-40, 8388607.5, 8388609.0], F32)])
    x = np.concatenate([x, -x])
    c = np.copysign(F32(0.49999997), x).astype(F32)
    trick = np.trunc((x + c).astype(F32))                      # float32 add, then truncate
    want = (np.sign(x) * np.floor(np.abs(x.astype(np.float64)) + 0.5)).astype(F32)  # half away from zero
    assert np.nextafter(F32(0.5), F32(0)) == F32(0.49999997)
    assert np.array_equal(trick, want), x[trick != want][:8]


def test_q4_nibble_order_one_hot(orc, rng):
    """Element 2i is the low nibble of byte i, 2i+1 the high nibble."""
    qs = rng.integers(0, 256, 16, dtype=np.uint8)
    codes = ref.q4_codes(qs, 1, 32)[0]
    for j in range(32):
        a = np.zeros(32, np.int8)
        a[j] = 1
        assert orc.q4_block_isum(qs, a) == codes[j] - 8
        assert orc.q4_block_isum(qs, a, scalar=True) == codes[j] - 8


def test_q4_block_isum_brute_force(orc, rng):
    for _ in range(200):
        qs = rng.integers(0, 256, 16, dtype=np.uint8)
        a = rng.integers(-127, 128, 32).astype(np.int8)
        want = int(np.dot(ref.q4_codes(qs, 1, 32)[0] - 8, a.astype(np.int64)))
        assert orc.q4_block_isum(qs, a) == want
        assert orc.q4_block_isum(qs, a, scalar=True) == want
    # extremes: all codes 0 against -127 and all 15 against 127
    assert orc.q4_block_isum(np.zeros(16, np.uint8), np.full(32, -127, np.int8)) == 32 * 8 * 127
    assert orc.q4_block_isum(np.full(16, 0xFF, np.uint8), np.full(32, 127, np.int8)) == 32 * 7 * 127


def test_quantize_q4_roundtrip(orc, rng):
    x = rng.uniform(-1, 1, 32 * 40).astype(F32)
    x[:32] = 0.0  # d == 0 block -> 0x88 (tensor.rs:120-122)
    qs, sc = orc.quantize_q4(x)
    assert sc[0] == 0 and np.all(qs[:16] == 0x88)
    deq = orc.dequantize_q4(qs, sc, x.size)
    assert np.array_equal(deq, ref.dequant_q4(qs, sc, 1, x.size)[0].astype(F32))
    # reconstruction error bounded by one step (the +8.5 then truncation rounds)
    step = np.repeat(sc, 32)
    assert np.all(np.abs(deq - x) <= step * 0.5 + 1e-7)


# ---- GEMV (cpu.rs:49-111, 888-941) -----------------------------------------
@pytest.mark.parametrize("n,k", [(8, 32), (16, 128), (5, 256)])
def test_q4_gemv_exact(orc, rng, n, k):
    x = rng.uniform(-1, 1, k).astype(F32)
    qs = rng.integers(0, 256, n * k // 2, dtype=np.uint8)
    sc = rng.uniform(0.003, 0.006, n * k // 32).astype(F32)
    got = orc.matmul_transposed_q4(x[None], qs, sc, n)[0]
    want = ref.gemv_q4_exact_f32(x, qs, sc, n, k)
    assert np.array_equal(got, want)


def test_q4_gemv_vs_dequantised_f64(orc, rng):
    """test_opencl_matmul_q4_decoding (test/opencl.rs:237-258): M=1, K=128,
    N=64 against a dot over dequantised weights; the reference allows 1e-3,
    the Q8 activation rounding is the only difference."""
    m, k, n = 1, 128, 64
    a = rng.uniform(-1, 1, (m, k)).astype(F32)
    b = rng.uniform(-1, 1, (n, k)).astype(F32)
    qs, sc = orc.quantize_q4(b)
    got = orc.matmul_transposed_q4(a, qs, sc, n)
    want = a.astype(np.float64) @ ref.dequant_q4(qs, sc, n, k).T
    # Q8 activation error: |a_i - q_i d| <= d/2 per element
    assert np.max(np.abs(got - want)) < 0.1
    exact_act = ref.linear64(a, ref.dequant_q4(qs, sc, n, k))
    assert np.max(np.abs(got - exact_act)) < 1e-4


def test_q4_gemv_prefill_rows(orc, rng):
    """test_opencl_q4_prefill_stress (test/opencl.rs:475-510): M=4, K=256, N=128;
    each row is quantised and reduced exactly like M=1."""
    m, k, n = 4, 256, 128
    a = rng.uniform(-1, 1, (m, k)).astype(F32)
    qs = rng.integers(0, 256, n * k // 2, dtype=np.uint8)
    sc = rng.uniform(0.003, 0.006, n * k // 32).astype(F32)
    got = orc.matmul_transposed_q4(a, qs, sc, n)
    for i in range(m):
        assert np.array_equal(got[i], ref.gemv_q4_exact_f32(a[i], qs, sc, n, k))


def test_q8w_gemv_exact(orc, rng):
    n, k = 12, 96
    x = rng.uniform(-2, 2, k).astype(F32)
    w = rng.integers(-127, 128, n * k).astype(np.int8)
    sc = rng.uniform(2e-4, 3.5e-4, n * k // 32).astype(F32)
    got = orc.matmul_transposed_q8w(x[None], w, sc, n)[0]
    assert np.array_equal(got, ref.gemv_q8w_exact_f32(x, w, sc, n, k))


# ---- f32 matmuls (cpu.rs:114-269; test/cpu.rs:103-160) ---------------------
def test_matmul_f32(orc, rng):
    for (m, k, n) in [(1, 128, 256), (16, 64, 32)]:
        a = rng.uniform(-1, 1, (m, k)).astype(F32)
        b = rng.uniform(-1, 1, (k, n)).astype(F32)
        assert np.max(np.abs(orc.matmul(a, b) - a.astype(np.float64) @ b)) < 1e-4


def test_matmul_transposed_and_slice_f32(orc, rng):
    a = rng.uniform(-1, 1, (4, 128)).astype(F32)
    b = rng.uniform(-1, 1, (64, 128)).astype(F32)
    assert np.max(np.abs(orc.matmul_transposed_f32(a, b) - a.astype(np.float64) @ b.T)) < 1e-4
    q = rng.uniform(-1, 1, (1, 64)).astype(F32)
    kc = rng.uniform(-1, 1, (10, 64)).astype(F32)
    got = orc.matmul_slice(q, kc, 10)
    assert np.max(np.abs(got - q.astype(np.float64) @ kc.T)) < 1e-4
    # sequential f32 order (cpu.rs:548): exact emulation on one row
    s = F32(0)
    for i in range(64):
        s = F32(s + F32(q[0, i] * kc[3, i]))
    assert got[0, 3] == s


# ---- elementwise / row ops (test/cpu.rs:162-245) ---------------------------
def test_rms_norm_kat(orc):
    y = orc.rms_norm(np.array([[1, 2, 3, 4]], F32), np.ones(4, F32), 1e-5)[0]
    assert abs(y[0] - 0.3651) < 1e-3 and abs(y[3] - 1.4605) < 1e-3
    assert np.allclose(y, ref.rmsnorm64([1, 2, 3, 4], np.ones(4), 1e-5), rtol=1e-6)


def test_rms_norm_closed_form(orc, rng):
    x = rng.normal(0, 1, (3, 256)).astype(F32)
    w = rng.normal(1, 0.02, 256).astype(F32)
    assert np.allclose(orc.rms_norm(x, w, 1e-5), ref.rmsnorm64(x, w, 1e-5), rtol=1e-5, atol=1e-6)


def test_softmax_kat(orc):
    d = orc.softmax(np.array([[1, 2, 3]], F32))[0]
    assert abs(d.sum() - 1) < 1e-5 and d[2] > d[1] > d[0]
    e = np.exp(np.array([1, 2, 3.0]) - 3)
    assert np.allclose(d, e / e.sum(), rtol=1e-6)


def test_rope_kat(orc):
    """test_rope_inplace (test/cpu.rs:229-245): [1,0,0,1] at pos 1."""
    d = orc.rope_inplace(np.array([[1, 0, 0, 1]], F32), 1)[0]
    assert abs(np.hypot(d[0], d[2]) - 1) < 1e-5 and abs(np.hypot(d[1], d[3]) - 1) < 1e-5
    assert d[0] != 1.0
    assert np.allclose(d, ref.rope64([[1, 0, 0, 1]], 1)[0], atol=1e-6)


def test_rope_identity_at_zero_and_closed_form(orc, rng):
    x = rng.normal(0, 1, (5, 128)).astype(F32)
    assert np.array_equal(orc.rope_inplace(x[:1], 0), x[:1])
    got = orc.rope_inplace(x, 37)
    assert np.allclose(got, ref.rope64(x, 37), atol=2e-5)
    # pairs (j, j+hd/2) keep their norm
    n0 = np.hypot(x[:, :64], x[:, 64:])
    n1 = np.hypot(got[:, :64], got[:, 64:])
    assert np.allclose(n0, n1, rtol=1e-5)


def test_silu_mul_add_scale(orc, rng):
    g = rng.uniform(-1, 1, 25).astype(F32)
    u = rng.uniform(-1, 1, 25).astype(F32)
    g64 = g.astype(np.float64)
    assert np.allclose(orc.silu_mul(g, u), g64 / (1 + np.exp(-g64)) * u, atol=1e-6)
    assert np.array_equal(orc.add_assign(g, u), g + u)
    assert np.array_equal(orc.scale(g, 0.125), g * F32(0.125))


def test_f16_rounding(orc, rng):
    vals = np.concatenate([rng.normal(0, 3, 500), [0.0, -0.0, 65504.0, 65520.0, 1e-8, 6e-5, 1.0009765625]])
    for v in vals.astype(F32):
        assert orc.f32_to_f16_bits(float(v)) == int(np.array(v, F32).astype(np.float16).view(np.uint16))


def test_argmax_lowest_index_on_ties(orc):
    i, m = orc.argmax(np.array([1, 5, 5, 2], F32))
    assert i == 1 and m == 0.0
    i, m = orc.argmax(np.array([3, 1, 2], F32))
    assert i == 0 and m == 1.0


# ---- the aarch64 restatement (orc_set_arch(1)) ------------------------------
# Known answers worked out by hand from the NEON code's order, on inputs whose
# products are exact, so that only the order of additions (and fusing)
# decides the result; the x86 build gives a different value on each.

def _with_arch(orc, arch, fn):
    orc.set_arch(arch)
    try:
        return fn()
    finally:
        orc.set_arch(0)


def test_neon_dot_pairs_accumulators(orc):
    """simd_dot_f32 on aarch64 (cpu.rs:518-521, 535): elements 0, 8 and 12
    sit in accumulators 0, 2 and 3 (lane 0); (s0 + s1) + (s2 + s3) adds the
    two ones before they meet 2^24, so the sum is 2^24 + 2.  In sequence
    each +1 on 2^24 rounds back to 2^24."""
    a = np.zeros((1, 32), F32)
    a[0, 0], a[0, 8], a[0, 12] = 2.0 ** 24, 1.0, 1.0
    b = np.ones((1, 32), F32)
    neon = _with_arch(orc, 1, lambda: orc.matmul_slice(a, b, 1))[0, 0]
    x86 = orc.matmul_slice(a, b, 1)[0, 0]
    assert neon == 2.0 ** 24 + 2 and x86 == 2.0 ** 24


def test_neon_dot_fuses_multiply_add(orc):
    """vfmaq_f32 (cpu.rs:481): elements 0 and 32 share accumulator 0 lane 0;
    -1 + (1 + 2^-12)^2 fused keeps the 2^-24 term (2^-11 + 2^-24), unfused
    the product rounds it away (2^-11)."""
    a = np.zeros((1, 64), F32)
    b = np.zeros((1, 64), F32)
    a[0, 0], b[0, 0] = -1.0, 1.0
    a[0, 32] = b[0, 32] = 1.0 + 2.0 ** -12
    neon = _with_arch(orc, 1, lambda: orc.matmul_slice(a, b, 1))[0, 0]
    x86 = orc.matmul_slice(a, b, 1)[0, 0]
    assert neon == 2.0 ** -11 + 2.0 ** -24 and x86 == 2.0 ** -11


def test_neon_q4_gemv_adds_four_blocks_first(orc):
    """kernel_neon_sdot (cpu.rs:850): blocks 4 and 5 (one group) are summed
    before the running total 2^24 from block 0, giving 2^24 + 2; the x86
    block loop (cpu.rs:932) adds them one at a time and stays at 2^24.
    Block sums are 1 (one weight code 9 against activation code 1), scales
    d_w * d_a = 2^24 for block 0 and 1 otherwise."""
    nb = 8
    xq = np.zeros((1, 32 * nb), np.int8)
    for b in (0, 4, 5):
        xq[0, 32 * b] = 1
    xd = np.ones((1, nb), F32)
    xd[0, 0] = 2.0 ** 12
    qs = np.full(16 * nb, 0x88, np.uint8)    # every code 8: (q - 8) = 0
    qs[16 * np.arange(nb)] = 0x89            # element 0 of each block: code 9
    sc = np.ones(nb, F32)
    sc[0] = 2.0 ** 12
    neon = _with_arch(orc, 1, lambda: orc.gemv_codes(xq, xd, qs, sc, 1))[0, 0]
    x86 = orc.gemv_codes(xq, xd, qs, sc, 1)[0, 0]
    assert neon == 2.0 ** 24 + 2 and x86 == 2.0 ** 24


def test_neon_saxpy_fuses_over_whole_steps(orc):
    """simd_saxpy on aarch64 (cpu.rs:570): y = fma(alpha, x, y) over
    32-element steps, unfused for the leftovers (cpu.rs:610-615): through
    matmul (cpu.rs:198), y[0] = -1 + (1 + 2^-12)^2 keeps 2^-24 when fused;
    element 32 (a leftover of n = 33) does not."""
    a = np.array([[1.0, 1.0 + 2.0 ** -12]], F32)
    b = np.zeros((2, 33), F32)
    b[0, 0] = b[0, 32] = -1.0
    b[1, 0] = b[1, 32] = 1.0 + 2.0 ** -12
    neon = _with_arch(orc, 1, lambda: orc.matmul(a, b))[0]
    x86 = orc.matmul(a, b)[0]
    assert neon[0] == 2.0 ** -11 + 2.0 ** -24 and neon[32] == 2.0 ** -11
    assert x86[0] == 2.0 ** -11 and x86[32] == 2.0 ** -11


def test_gemv_codes_matches_matmul_transposed(orc, rng):
    """The probe entry (block loop on given codes) equals matmul_transposed,
    which quantises first, bit for bit."""
    m, n, k = 3, 40, 256
    a = rng.normal(0, 1, (m, k)).astype(F32)
    qs = rng.integers(0, 256, n * k // 2).astype(np.uint8)
    sc = rng.uniform(0.003, 0.006, n * k // 32).astype(F32)
    xq, xd = zip(*(orc.quantize_row_q8_0(a[i]) for i in range(m)))
    got = orc.gemv_codes(np.stack(xq), np.stack(xd), qs, sc, n)
    assert np.array_equal(got, orc.matmul_transposed_q4(a, qs, sc, n))
    w8 = rng.integers(-127, 128, n * k).astype(np.int8)
    got8 = orc.gemv_codes(np.stack(xq), np.stack(xd), w8, sc, n, q8w=True)
    assert np.array_equal(got8, orc.matmul_transposed_q8w(a, w8, sc, n))


def test_code_replay_checks_midpoints(orc):
    """orc_inject_codes: the oracle takes the given codes; a differing code
    passes only one step away from its own with x*inv at the rounding
    midpoint (within tol).  One block with amax 127 (d = 1, inv = 1): 2.5
    sits on the 2|3 midpoint, 2.2 does not."""
    x = np.zeros(32, np.float32)
    x[0], x[1], x[2] = 127.0, 2.5, 2.2
    own, d = orc.quantize_row_q8_0(x)
    assert own[1] == 3 and own[2] == 2 and d[0] == 1.0
    try:
        orc.inject_codes(own, 1e-3)  # its own codes: nothing differs
        q, _ = orc.quantize_row_q8_0(x)
        st = orc.injected_stats()
        assert np.array_equal(q, own) and st == {"taken": 32, "differ": 0, "bad": 0, "max_dist": 0.0}
        mid = own.copy()
        mid[1] = 2  # the other side of the 2.5 midpoint: taken, not bad
        orc.inject_codes(mid, 1e-3)
        q, _ = orc.quantize_row_q8_0(x)
        st = orc.injected_stats()
        assert q[1] == 2 and st["differ"] == 1 and st["bad"] == 0 and st["max_dist"] == 0.0
        for i, c in ((2, 3), (1, 1)):  # 2.2 is 0.3 from a midpoint; 1 is two steps from 3
            bad = own.copy()
            bad[i] = c
            orc.inject_codes(bad, 1e-3)
            q, _ = orc.quantize_row_q8_0(x)
            st = orc.injected_stats()
            assert q[i] == c and st["differ"] == 1 and st["bad"] == 1
        orc.inject_codes(own[:16], 1e-3)  # fewer codes than asked for
        orc.quantize_row_q8_0(x)
        assert orc.injected_stats()["bad"] == 16
    finally:
        orc.inject_codes(None)
    q, _ = orc.quantize_row_q8_0(x)
    assert np.array_equal(q, own)

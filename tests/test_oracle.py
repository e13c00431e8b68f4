"""Pin the CPU oracle (oracle/cpu_ref.c) before trusting it as the checker.

Each check is chosen so that a plausible restatement mistake fails it:
  * bf16 conversion: against torch's RNE bf16 cast, including exact ties.
  * unpacking: one-hot words and exhaustive codes at every position (a wrong
    word index, shift or mask changes the decoded value).
  * group indexing: distinct power-of-two scales per group.
  * dequant rounding: float(q)*s is exact, so q*s+b has one rounding; checked
    against the fp64 evaluation rounded once to fp32.
  * GEMV / GEMM sums: closed forms (s=1, b=0 gives the code sums) and an
    independent torch fp64 matmul of the dequantised matrix.
"""
import numpy as np
import pytest
import torch

import oracle
from miori_amd import synth


def test_bf16_rne_matches_torch():
    rng = np.random.default_rng(1)
    f = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-20, 20, 20000).astype(np.float32),
        # exact ties: low 16 bits = 0x8000 with even and odd kept LSB
        (np.array([0x3F808000, 0x3F818000, 0xBF808000, 0x40490000, 0x3F80FFFF, 0x00008000],
                  dtype=np.uint32)).view(np.float32),
        np.array([0.0, -0.0, 1.0, -1.0, 3.4e38, -3.4e38, 1e-40], dtype=np.float32),
    ])
    got = oracle.f32_to_bf16(f)
    want = torch.from_numpy(f).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(got, want)
    # the generator's vectorised rounding agrees with the oracle
    np.testing.assert_array_equal(synth.f32_to_bf16_bits(f), got)


def test_bf16_to_f32_matches_torch():
    bits = np.arange(0, 65536, 7, dtype=np.uint16)
    bits = bits[(bits & 0x7F80) != 0x7F80]  # finite values
    want = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(oracle.bf16_to_f32(bits), want)
    assert oracle._load().orc_bf16_to_f32(0x3FC0) == 1.5


def _unit_scales(N, K, G):
    one = np.full((N, K // G), 0x3F80, dtype=np.uint16)   # bf16 1.0
    zero = np.zeros((N, K // G), dtype=np.uint16)
    return one, zero


@pytest.mark.parametrize("bits", [4, 8])
def test_unpack_exhaustive_codes(bits):
    """Every code value at every position of a word decodes to itself."""
    per = 32 // bits
    ncode = 1 << bits
    K, G = 32, 32
    N = ncode
    q = np.zeros((N, K // per), dtype=np.uint32)
    for n in range(N):
        for w in range(K // per):
            v = 0
            for j in range(per):
                v |= ((n + 3 * (w * per + j)) % ncode) << (bits * j)
            q[n, w] = v
    s, b = _unit_scales(N, K, G)
    deq = oracle.dequant_f32(q, s, b, bits, K, G)
    want = np.array([[(n + 3 * k) % ncode for k in range(K)] for n in range(N)], dtype=np.float32)
    np.testing.assert_array_equal(deq, want)


@pytest.mark.parametrize("bits", [4, 8])
def test_unpack_one_hot(bits):
    """A single non-zero code at position k appears only at element k."""
    per = 32 // bits
    K, G = 64, 32
    top = (1 << bits) - 1
    s, b = _unit_scales(1, K, G)
    for k in range(K):
        q = np.zeros((1, K // per), dtype=np.uint32)
        q[0, k // per] = np.uint32(top << (bits * (k % per)))
        deq = oracle.dequant_f32(q, s, b, bits, K, G)[0]
        want = np.zeros(K, dtype=np.float32)
        want[k] = top
        np.testing.assert_array_equal(deq, want)
        assert oracle.dequant4_elem(q, s, b, 0, k, K, G) == top if bits == 4 else \
            oracle.dequant8_elem(q, s, b, 0, k, K, G) == top


@pytest.mark.parametrize("G", [32, 64, 128])
def test_group_indexing(G):
    """Scale of group g = 2^-(g + 3n): a wrong group or row stride shows."""
    N, K = 3, 256
    ng = K // G
    q = np.full((N, K // 8), 0x11111111, dtype=np.uint32)  # every nibble = 1
    s = synth.f32_to_bf16_bits(np.array([[2.0 ** -(g + 3 * n) for g in range(ng)]
                                         for n in range(N)], dtype=np.float32))
    b = np.zeros_like(s)
    deq = oracle.dequant_f32(q, s, b, 4, K, G)
    want = np.array([[2.0 ** -(k // G + 3 * n) for k in range(K)] for n in range(N)], dtype=np.float32)
    np.testing.assert_array_equal(deq, want)


@pytest.mark.parametrize("bits", [4, 8])
def test_dequant_single_rounding(bits):
    """float(q)*s is exact, so the fp32 dequant equals fp64 q*s+b rounded once."""
    w = synth.quant_weights(64, 256, 64, bits, seed=11)
    deq = oracle.dequant_f32(w.q, w.s, w.b, bits, 256, 64)
    per = 32 // bits
    mask = (1 << bits) - 1
    codes = np.stack([(w.q >> np.uint32(bits * j)) & np.uint32(mask) for j in range(per)], axis=-1)
    codes = codes.reshape(64, 256).astype(np.float64)
    sf = np.repeat(synth.bf16_bits_to_f32(w.s).astype(np.float64), 64, axis=1)
    bf = np.repeat(synth.bf16_bits_to_f32(w.b).astype(np.float64), 64, axis=1)
    assert np.all(codes * sf == (codes * sf).astype(np.float32))  # product exact in fp32
    want = (codes * sf + bf).astype(np.float32)
    np.testing.assert_array_equal(deq, want)
    # bf16 dequant = RNE of the fp32 value
    np.testing.assert_array_equal(oracle.dequant_bf16(w.q, w.s, w.b, bits, 256, 64),
                                  synth.f32_to_bf16_bits(want))


@pytest.mark.parametrize("bits", [4, 8])
def test_gemv_closed_form(bits):
    """s=1, b=0, x=1: y[n] is the sum of the codes of row n."""
    N, K, G = 16, 512, 64
    w = synth.quant_weights(N, K, G, bits, seed=5)
    s, b = _unit_scales(N, K, G)
    x = np.full((1, K), 0x3F80, dtype=np.uint16)
    y = oracle.gemv_f64(w.q, s, b, x, bits, K, G)[0]
    per, mask = 32 // bits, (1 << bits) - 1
    want = sum(((w.q >> np.uint32(bits * j)) & np.uint32(mask)).astype(np.int64).sum(axis=1)
               for j in range(per))
    np.testing.assert_array_equal(y, want.astype(np.float64))


@pytest.mark.parametrize("bits,M", [(4, 1), (4, 3), (8, 2)])
def test_gemv_matches_torch_fp64(bits, M):
    N, K, G = 48, 384, 64 if bits == 4 else 32
    w = synth.quant_weights(N, K, G, bits, seed=21 + M)
    x = synth.activations(M, K, seed=99)
    y = oracle.gemv_f64(w.q, w.s, w.b, x, bits, K, G)
    Wd = torch.from_numpy(oracle.dequant_f32(w.q, w.s, w.b, bits, K, G).astype(np.float64))
    X = torch.from_numpy(synth.bf16_bits_to_f32(x).astype(np.float64))
    np.testing.assert_allclose(y, (X @ Wd.T).numpy(), rtol=1e-12, atol=1e-12)
    # threaded evaluation is the same arithmetic per row
    np.testing.assert_array_equal(y, oracle.gemv_f64(w.q, w.s, w.b, x, bits, K, G, nthreads=4))
    # row-range evaluation agrees on its rows
    yr = oracle.gemv_rows_f64(w.q, w.s, w.b, x, bits, K, G, 5, 17)
    np.testing.assert_array_equal(yr[:, 5:17], y[:, 5:17])


def test_gemm_matches_torch_fp64():
    rng = np.random.default_rng(3)
    A = synth.f32_to_bf16_bits(rng.standard_normal((37, 96)).astype(np.float32))
    B = synth.f32_to_bf16_bits(rng.standard_normal((20, 96)).astype(np.float32))
    rows = np.array([0, 5, 36], dtype=np.int64)
    C = oracle.gemm_bf16_f64(A, B, rows)
    At = torch.from_numpy(synth.bf16_bits_to_f32(A).astype(np.float64))
    Bt = torch.from_numpy(synth.bf16_bits_to_f32(B).astype(np.float64))
    np.testing.assert_allclose(C, (At @ Bt.T).numpy()[rows], rtol=1e-12, atol=1e-12)


def test_reference_test_gemm_inputs():
    """The reference's test-gemm operands (src/main.cpp:578-602: M=4, N=8,
    K=32, lda=64, ldb=32, A[i]=bf16(sin(0.13 i)), B[i]=bf16(cos(0.17 i)))
    against an fp32-accumulated loop as that test does it."""
    M, N, K, lda, ldb = 4, 8, 32, 64, 32
    a = synth.f32_to_bf16_bits(np.sin(np.arange(M * lda, dtype=np.float32) * np.float32(0.13)))
    b = synth.f32_to_bf16_bits(np.cos(np.arange(N * ldb, dtype=np.float32) * np.float32(0.17)))
    A = np.ascontiguousarray(a.reshape(M, lda)[:, :K])
    B = np.ascontiguousarray(b.reshape(N, ldb)[:, :K])
    C = oracle.gemm_bf16_f64(A, B)
    af, bf_ = synth.bf16_bits_to_f32(A), synth.bf16_bits_to_f32(B)
    ref32 = np.zeros((M, N), dtype=np.float32)
    for k in range(K):
        ref32 += af[:, k:k + 1] * bf_[:, k][None, :]
    np.testing.assert_allclose(C, ref32, rtol=0, atol=1e-5)


def test_synth_distributions():
    w = synth.quant_weights(512, 2048, 64, 4, seed=1)
    sf = synth.bf16_bits_to_f32(w.s)
    assert 0.00099 <= sf.min() and sf.max() <= 0.0101
    bf = synth.bf16_bits_to_f32(w.b).astype(np.float64)
    resid = bf + 8.0 * sf
    assert abs(resid.std() - 1e-3) < 2e-4
    nib = np.concatenate([((w.q >> np.uint32(4 * j)) & np.uint32(15)).ravel() for j in range(8)])
    counts = np.bincount(nib, minlength=16) / nib.size
    assert np.all(np.abs(counts - 1 / 16) < 2e-3)
    x = synth.bf16_bits_to_f32(synth.activations(4, 4096))
    assert abs(x.mean()) < 0.05 and abs(x.std() - 1.0) < 0.05
    w8 = synth.quant_weights(64, 2048, 64, 8, seed=2)
    s8 = synth.bf16_bits_to_f32(w8.s)
    assert 1e-4 * 0.99 <= s8.min() and s8.max() <= 1e-3 * 1.01
    np.testing.assert_array_equal(synth.bf16_bits_to_f32(w8.b), (np.float32(-128) * s8))
    # determinism
    np.testing.assert_array_equal(synth.quant_weights(8, 64, 32, 4, seed=9).q,
                                  synth.quant_weights(8, 64, 32, 4, seed=9).q)


# ---- gemm_naive oracle (shaders/ops.metal:199-251; check src/main.cpp:578-602)

def _bf(vals):
    return synth.f32_to_bf16_bits(np.asarray(vals, dtype=np.float32))


def test_naive_order_is_sequential_fp32():
    """The definition is the k-ordered fp32 chain: 1 + 2^24 rounds back to 2^24
    (tie to even), so [1, 2^24, -2^24] sums to 0 forwards while the exact
    sum, and the reversed order, give 1. bf16 x bf16 products are exact in
    fp32, so this pins the order and nothing else can differ."""
    A = _bf([1.0, 4096.0, -4096.0])
    B = _bf([1.0, 4096.0, 4096.0])
    assert oracle.gemm_naive_f32(A, B, 1, 1, 3, 3, 3, 1)[0] == 0.0
    assert oracle.gemm_naive_f32(A[::-1].copy(), B[::-1].copy(), 1, 1, 3, 3, 3, 1)[0] == 1.0


def test_naive_integer_closed_form_with_strides():
    """Small integers: every product and partial sum is exact, so the result
    is the exact integer product. Strides, padding and the B^T orientation
    are all pinned (a transposed operand or wrong stride changes the sums)."""
    rng = np.random.default_rng(3)
    M, N, K, lda, ldb, ldc = 5, 7, 40, 48, 43, 9
    Ai = rng.integers(-8, 9, size=(M, lda))
    Bi = rng.integers(-8, 9, size=(N, ldb))
    C = oracle.gemm_naive_f32(_bf(Ai), _bf(Bi), M, N, K, lda, ldb, ldc).reshape(M, ldc)
    exact = Ai[:, :K] @ Bi[:, :K].T
    np.testing.assert_array_equal(C[:, :N], exact.astype(np.float32))
    assert np.all(C[:, N:] == 0.0)  # outside the output columns nothing is written


def test_naive_reference_case_vs_fp64():
    """The reference's test-gemm inputs (src/main.cpp:578-602): M=4, N=8,
    K=32, lda=64, ldb=32, ldc=16, a_i = bf16(sin(0.13 i)), b_i = bf16(cos(0.17 i));
    the fp32 chain is within fp32 rounding of the fp64 product."""
    M, N, K, lda, ldb, ldc = 4, 8, 32, 64, 32, 16
    a = _bf(np.sin(np.arange(M * lda, dtype=np.float32) * np.float32(0.13)))
    b = _bf(np.cos(np.arange(N * ldb, dtype=np.float32) * np.float32(0.17)))
    C = oracle.gemm_naive_f32(a, b, M, N, K, lda, ldb, ldc).reshape(M, ldc)[:, :N]
    af = synth.bf16_bits_to_f32(a).astype(np.float64).reshape(M, lda)[:, :K]
    bf = synth.bf16_bits_to_f32(b).astype(np.float64).reshape(N, ldb)[:, :K]
    np.testing.assert_allclose(C, af @ bf.T, rtol=0, atol=1e-5)


# ---- fused decode-op transforms (shaders/ops.metal:86-114 rmsnorm, :129-139 silu_mul)

def _bf_ulp_diff(a_bits, b_bits):
    a = a_bits.astype(np.int32)
    b = b_bits.astype(np.int32)
    return np.abs(a - b)


def test_rmsnorm_closed_form():
    """x = 2 everywhere: sum(x^2)/K = 4 exactly, rsqrt(4 + 0) = 0.5 exactly, so
    h = bf16(1 * w) = w bit for bit. A sum instead of a mean, or a missing
    square, breaks it."""
    K = 2048
    w = synth.activations(1, K, seed=5).ravel()
    h = oracle.rmsnorm_bf16(np.full(K, 2.0, np.float32), w, 0.0)
    np.testing.assert_array_equal(h, w)


def test_rmsnorm_vs_torch_fp64():
    K = 2048
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(K) * 3).astype(np.float32)
    w = _bf(rng.standard_normal(K) * 0.2 + 1.0)
    h = oracle.rmsnorm_bf16(x, w, 1e-5)
    xt = torch.tensor(x, dtype=torch.float64)
    ref = xt / torch.sqrt((xt * xt).mean() + 1e-5) * torch.tensor(synth.bf16_bits_to_f32(w), dtype=torch.float64)
    ref_bits = synth.f32_to_bf16_bits(ref.float().numpy())
    d = _bf_ulp_diff(h, ref_bits)
    assert d.max() <= 1 and (d == 0).mean() > 0.98


def test_silu_mul_vs_torch_fp64_and_limits():
    rng = np.random.default_rng(2)
    g = (rng.standard_normal(4096) * 4).astype(np.float32)
    u = (rng.standard_normal(4096)).astype(np.float32)
    a = oracle.silu_mul_bf16(g, u)
    ref = torch.nn.functional.silu(torch.tensor(g, dtype=torch.float64)) * torch.tensor(u, dtype=torch.float64)
    d = _bf_ulp_diff(a, synth.f32_to_bf16_bits(ref.float().numpy()))
    assert d.max() <= 1 and (d == 0).mean() > 0.98
    # silu(0) = 0, silu(g) -> g for large g, silu(-g) -> 0 for large g
    lim = oracle.silu_mul_bf16(np.array([0.0, 40.0, -40.0], np.float32), np.ones(3, np.float32))
    v = synth.bf16_bits_to_f32(lim)
    assert v[0] == 0.0 and v[1] == 40.0 and abs(v[2]) < 1e-15

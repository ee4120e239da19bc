"""The MLP GEMM op (DGEN_HIP_K_GEMM) in both product modes against fp64
matrix products: every operand layout, every epilogue (bias, bias + tanh,
tanh gradient with per-tile column partials, weighted by input columns),
split-K partial sums, ragged shapes that take the bounds-checked loads and
aligned shapes that take the unchecked ones.

The split-bf16 mode (three bfloat16 parts per operand, six partial
products in fp32) must be as accurate as the fp32 matrix cores: its
relative L2 error against fp64 is held to twice the fp32 mode's own error
on the same operands (plus 1e-7 for the cases where both are near zero).
Needs a GPU."""
import numpy as np
import pytest

from dgen_hip import runtime as R
from dgen_hip.program import Program

pytestmark = pytest.mark.gpu

TILE = 128


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def run_gemm(mode, M, N, K, alay, blay, epi, split=1, colsum=False, nw=0, seed=0, pad=0, planes=False):
    """One GEMM op (with planes: B split into bfloat16 planes by a
    DGEN_HIP_K_SPLIT_BF16 op first); returns (C, column partials or None)
    and the fp64 reference of both."""
    rng = np.random.default_rng(seed)
    lda = (K if alay == 0 else M) + pad
    ldb = (N if blay == 0 else K) + pad
    ldc = N + pad
    A = rng.standard_normal(((M if alay == 0 else K), lda)).astype(np.float32)
    B = (rng.standard_normal(((K if blay == 0 else N), ldb)) / np.sqrt(K)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    aux = np.tanh(rng.standard_normal((M, ldc))).astype(np.float32)
    X = rng.standard_normal((M, max(nw, 1))).astype(np.float32)
    opA = (A[:, :K] if alay == 0 else A[:, :M].T).astype(np.float64)
    opB = (B[:, :N] if blay == 0 else B[:, :K].T).astype(np.float64)
    ref = opA @ opB
    if epi == R.EPI_BIAS:
        ref = ref + bias
    elif epi == R.EPI_BIAS_TANH:
        ref = np.tanh(ref + bias)
    elif epi == R.EPI_TANH_GRAD:
        h = aux[:, :N].astype(np.float64)
        ref = ref * (1.0 - h * h)
    mt = (M + TILE - 1) // TILE
    ref_cs = None
    if colsum:
        rows = []
        for t in range(mt):
            blk = ref[t * TILE:(t + 1) * TILE]
            xb = X[t * TILE:(t + 1) * TILE].astype(np.float64)
            rows += [xb[:, q] @ blk for q in range(nw)] + [blk.sum(0)]
        ref_cs = np.array(rows)

    p = Program(max_frames=1)
    cA = p.alloc("A", A.size)
    cB = p.alloc("B", B.size)
    cC = p.alloc("C", M * ldc)
    cb = p.alloc("bias", N)
    ca = p.alloc("aux", aux.size)
    kchunk = -(-K // split)
    kchunk = -(-kchunk // 16) * 16
    splits = -(-K // kchunk)
    cw = p.alloc("ws", max(1, splits * M * N))
    ccs = p.alloc("colsum", max(1, mt * (nw + 1) * N))
    cx = p.alloc("X", X.size)
    cp = -1
    if planes:
        k8 = -(-K // 8)
        cp = p.alloc("planes", 3 * k8 * N * 4)
        # op(B) as [K][N]: B[k][n] (layout 0) or B[n][k] (layout 1)
        ldk, ldn = (ldb, 1) if blay == 0 else (1, ldb)
        p.add(R.K_SPLIT_BF16, [cB, cp, K, N, ldk, ldn], label="split")
    args = [cA, cB, cC, M, N, K, lda, ldb, ldc, alay, blay, epi,
            cb if epi in (R.EPI_BIAS, R.EPI_BIAS_TANH) else -1,
            ca if epi == R.EPI_TANH_GRAD else -1, ldc, split, cw if split > 1 else 0,
            ccs if colsum else -1, cx if nw else -1, nw, mode, cp]
    p.add(R.K_GEMM, args, label="gemm")
    with R.HIPLazyRuntime(p, 0) as rt:
        rt.write("A", A)
        rt.write("B", B)
        rt.write("bias", bias)
        rt.write("aux", aux)
        rt.write("X", X)
        rt.runNoCopy()
        C = rt.read("C").reshape(M, ldc)[:, :N]
        cs = rt.read("colsum")[:mt * (nw + 1) * N].reshape(mt * (nw + 1), N) if colsum else None
    return C, cs, ref, ref_cs


CASES = {
    # name: (M, N, K, a_layout, b_layout, epilogue, split, column partials, nw, pad)
    "forward layer, aligned": (512, 512, 512, 0, 0, R.EPI_BIAS_TANH, 1, False, 0, 0),
    "heads, 127 columns": (1024, 127, 512, 0, 0, R.EPI_BIAS, 1, False, 0, 0),
    "data gradient, B transposed": (512, 256, 384, 0, 1, R.EPI_TANH_GRAD, 1, True, 0, 0),
    "first-layer partials": (384, 256, 128, 0, 1, R.EPI_TANH_GRAD, 1, True, 2, 0),
    "weight gradient, split-K": (256, 256, 4096, 1, 0, R.EPI_NONE, 8, False, 0, 0),
    "heads weight gradient": (512, 127, 4000, 1, 0, R.EPI_NONE, 5, False, 0, 0),
    "both transposed": (256, 384, 256, 1, 1, R.EPI_NONE, 1, False, 0, 0),
    "ragged": (200, 99, 53, 0, 0, R.EPI_BIAS, 1, False, 0, 3),
    "ragged, k-major": (130, 129, 77, 1, 1, R.EPI_TANH_GRAD, 1, True, 1, 1),
    "ragged split-K": (300, 70, 1001, 1, 0, R.EPI_NONE, 3, False, 0, 2),
}


@pytest.mark.parametrize("name", list(CASES))
def test_split_bf16_products_are_as_accurate_as_fp32(gpu, name):
    M, N, K, al, bl, epi, split, colsum, nw, pad = CASES[name]
    print(f"gemm {name}: M={M} N={N} K={K} layouts {al}{bl} epi {epi} split {split}", flush=True)
    c32, cs32, ref, ref_cs = run_gemm(0, M, N, K, al, bl, epi, split, colsum, nw, pad=pad)
    c6, cs6, _, _ = run_gemm(1, M, N, K, al, bl, epi, split, colsum, nw, pad=pad)
    cp, csp, _, _ = run_gemm(1, M, N, K, al, bl, epi, split, colsum, nw, pad=pad, planes=True)
    e32, e6, ep = rel(c32, ref), rel(c6, ref), rel(cp, ref)
    print(f"  C rel L2 vs fp64: fp32 {e32:.3e} split-bf16 {e6:.3e} (B pre-split {ep:.3e})")
    assert e32 < 1e-5, e32
    assert e6 <= 2.0 * e32 + 1e-7, (e6, e32)
    # the planes are the same split: the products and sums are identical
    np.testing.assert_array_equal(cp, c6)
    if colsum:
        f32, f6 = rel(cs32, ref_cs), rel(cs6, ref_cs)
        print(f"  column partials: fp32 {f32:.3e} split-bf16 {f6:.3e}")
        assert f32 < 1e-5 and f6 <= 2.0 * f32 + 1e-7, (f6, f32)
        np.testing.assert_array_equal(csp, cs6)


def _bf16_to_f32(u16):
    return (u16.astype(np.uint32) << 16).view(np.float32)


def test_split_planes_sum_to_the_fp32_values_exactly(gpu):
    """x = h + m + l bit for bit for every value (normal, small, huge, signed
    zero, powers of two, values with all 24 significant bits set; values
    whose low part would be a bfloat16 subnormal, |x| < 2^-110, are outside
    what this pins), zero planes past K, and the layout (p*K8 + k/8)*N + n,
    element k%8."""
    rng = np.random.default_rng(7)
    K, N = 45, 19
    vals = np.concatenate([rng.standard_normal(300), rng.standard_normal(200) * 1e-20, rng.standard_normal(100) * 1e30,
                           [0.0, -0.0, 1.0, -2.0 ** -126, 2.0 ** 100, np.float32(1) - np.float32(2.0 ** -24)]])
    x = np.resize(vals, K * N).astype(np.float32)
    x[::7] = (np.float32(1.0) + np.float32(2.0 ** -23) * (np.arange(len(x[::7])) % 255 + 1)).astype(np.float32)
    src = x.reshape(K, N)
    p = Program(max_frames=1)
    cs = p.alloc("src", K * N)
    k8 = -(-K // 8)
    cp = p.alloc("planes", 3 * k8 * N * 4)
    p.add(R.K_SPLIT_BF16, [cs, cp, K, N, N, 1], label="split")
    with R.HIPLazyRuntime(p, 0) as rt:
        rt.write("src", src.reshape(-1))
        rt.runNoCopy()
        raw = rt.read("planes").view(np.uint16).reshape(3, k8, N, 8)
    parts = _bf16_to_f32(raw).astype(np.float64)  # [p][kg][n][j]
    total = parts.sum(0).transpose(0, 2, 1).reshape(k8 * 8, N)  # [k][n]
    np.testing.assert_array_equal(total[:K], src.astype(np.float64))
    assert not np.any(total[K:])
    # h is the round-to-nearest bfloat16 of x
    h = parts[0].transpose(0, 2, 1).reshape(k8 * 8, N)[:K]
    rne = (((src.view(np.uint32).astype(np.uint64) + 0x7FFF + ((src.view(np.uint32) >> 16) & 1)) >> 16) << 16)
    np.testing.assert_array_equal(h, rne.astype(np.uint32).view(np.float32).astype(np.float64))


def test_fp32_ops_written_without_the_planes_argument_still_run(gpu):
    """An fp32-product op built before arg[21] existed (left 0, as the op
    builder pads) configures and computes as before."""
    rng = np.random.default_rng(3)
    A = rng.standard_normal((128, 64)).astype(np.float32)
    B = rng.standard_normal((64, 128)).astype(np.float32)
    p = Program(max_frames=1)
    ca, cb, cc = p.alloc("A", A.size), p.alloc("B", B.size), p.alloc("C", 128 * 128)
    p.add(R.K_GEMM, [ca, cb, cc, 128, 128, 64, 64, 128, 128, 0, 0, R.EPI_NONE, -1, -1, 128, 1, 0, -1, -1, 0, 0],
          label="gemm")
    assert p.ops[0].arg[21] == 0
    with R.HIPLazyRuntime(p, 0) as rt:
        rt.write("A", A)
        rt.write("B", B)
        rt.runNoCopy()
        C = rt.read("C").reshape(128, 128)
    assert rel(C, A.astype(np.float64) @ B) < 1e-5


def test_product_mode_is_validated(gpu):
    p = Program(max_frames=1)
    a = p.alloc("A", 16 * 16)
    p.add(R.K_GEMM, [a, a, a, 16, 16, 16, 16, 16, 16, 0, 0, R.EPI_NONE, -1, -1, 16, 1, 0, -1, -1, 0, 2], label="gemm")
    with pytest.raises(Exception):
        with R.HIPLazyRuntime(p, 0) as rt:
            rt.runNoCopy()

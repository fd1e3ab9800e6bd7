"""GPU parity of the W8A8 int8 MFMA GEMM (lq_gemm_w8a8) through the C ABI.

* int32 accumulators: bit-exact against the oracle's int64 brute force on every kernel
  path (skinny M <= 64; LDS-DMA 256x256, 256x128 and 128x128 tiles; register-staged 128x128 tiles
  with and without split-K; generic);
* every epilogue kind (f32, f16, requantized int8 / uint8 / int16 / uint8-as-int8,
  fake-quantized f32) with activation and weight zero points, bias and ReLU: bit-exact
  against the oracle's epilogue (same op order, no FMA);
* BASELINE sizes (4096^3, 4096x11008): size-independent properties -- every row sum and
  column sum of C against A @ colsum(B) and B @ colsum(A) in int64, plus sampled rows
  exactly.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu


def _dev(L, arr):
    return L.tensor(np.ascontiguousarray(arr), device="gpu")


_OUT_DT = {O.OUT_I32: np.int32, O.OUT_F32: np.float32, O.OUT_F16: np.float16, O.OUT_Q8: np.int8,
           O.OUT_QU8: np.uint8, O.OUT_FQ32: np.float32, O.OUT_Q16: np.int16, O.OUT_QU8S8: np.int8}


def pack_weights(L, B):
    """B [N, K] int8 -> device buffer in the MFMA-packed layout (lq_pack_weights_i8)."""
    from lucid_amd import _C

    N, K = B.shape
    dB = _dev(L, B)
    nbytes = _C.lib().lq_packed_weights_size(N, K)
    dP = L.empty((max(nbytes, 16),), np.int8, "gpu")
    _C.call("lq_pack_weights_i8", dB.data_ptr(), K, N, K, dP.data_ptr(), None)
    return dP


def packed_layout_oracle(B):
    """The packed layout restated in numpy (tile (t, s), chunk l = row 16t + l%16,
    K-bytes 64s + 16(l//16) .. +15, zero padded)."""
    N, K = B.shape
    NT, KS = -(-N // 16), -(-K // 64)
    Bp = np.zeros((NT * 16, KS * 64), np.int8)
    Bp[:N, :K] = B
    t = Bp.reshape(NT, 16, KS, 4, 16)            # [t, row, s, g, byte]
    return np.ascontiguousarray(t.transpose(0, 2, 3, 1, 4)).reshape(-1)  # [t, s, g, row, byte]


def run_gemm(L, A, B, out_kind=O.OUT_I32, a_scale=None, b_scale=None, za=None, zb=None,
             b_sums=None, bias=None, out_scale=None, out_zp=None, qmin=-128, qmax=127,
             relu=False, lda=None, ldb=None, ldc=None, workspace=True, packed=False,
             flags=0):
    """Run lq_gemm_w8a8 (or lq_gemm_w8a8_packed) on host arrays; returns C [M, N]."""
    from lucid_amd import _C

    M, K = A.shape
    N = B.shape[0]
    lda = lda or K
    ldb = ldb or K
    ldc = ldc or N
    Ap = np.zeros((M, lda), np.int8)
    Ap[:, :K] = A
    Bp = np.zeros((N, ldb), np.int8)
    Bp[:, :K] = B
    dA, dB = _dev(L, Ap), _dev(L, Bp)
    dC = L.empty((M, ldc), _OUT_DT[out_kind], "gpu")
    keep = []

    def opt(a, dt=np.float32):
        if a is None:
            return None
        t = _dev(L, np.asarray(a, dt))
        keep.append(t)
        return t.data_ptr()

    sa = None if a_scale is None else np.atleast_1d(np.asarray(a_scale, np.float32))
    sb = None if b_scale is None else np.atleast_1d(np.asarray(b_scale, np.float32))
    ws_bytes = _C.lib().lq_gemm_w8a8_workspace_size(M, N, K) if workspace else 0
    ws = L.empty((max(ws_bytes, 1),), np.uint8, "gpu") if workspace else None
    if packed:
        dP = pack_weights(L, B)
        _C.call("lq_gemm_w8a8_packed", dA.data_ptr(), lda, dP.data_ptr(), dC.data_ptr(), ldc, M, N,
                K, opt(sa), 0 if sa is None or sa.size == 1 else 1, opt(sb),
                0 if sb is None or sb.size == 1 else 1,
                opt(None if za is None else [za]), opt(zb), opt(b_sums, np.int32), opt(bias),
                opt(None if out_scale is None else [out_scale]),
                opt(None if out_zp is None else [out_zp]), qmin, qmax, out_kind, (1 if relu else 0) | flags,
                ws.data_ptr() if ws is not None else None, ws_bytes, None)
        return dC.numpy()[:, :N]
    _C.call("lq_gemm_w8a8", dA.data_ptr(), lda, dB.data_ptr(), ldb, dC.data_ptr(), ldc, M, N, K,
            opt(sa), 0 if sa is None or sa.size == 1 else 1, opt(sb),
            0 if sb is None or sb.size == 1 else 1,
            opt(None if za is None else [za]), opt(zb), opt(b_sums, np.int32), opt(bias),
            opt(None if out_scale is None else [out_scale]),
            opt(None if out_zp is None else [out_zp]), qmin, qmax, out_kind, (1 if relu else 0) | flags,
            ws.data_ptr() if ws is not None else None, ws_bytes, None)
    return dC.numpy()[:, :N]


KINDS = [O.OUT_F32, O.OUT_F16, O.OUT_Q8, O.OUT_QU8, O.OUT_FQ32, O.OUT_Q16, O.OUT_QU8S8, O.OUT_I32]
GRID = {O.OUT_Q8: (-128, 127), O.OUT_QU8: (0, 255), O.OUT_FQ32: (0, 255), O.OUT_Q16: (0, 255),
        O.OUT_QU8S8: (0, 255)}


def _codes(rng, shape, lo=-127, hi=127):
    return rng.integers(lo, hi + 1, size=shape, dtype=np.int64).astype(np.int8)


# Shapes chosen to hit every dispatch path of the kernel selector:
#   M <= 16 / 32 / 64 -> skinny (1, 2, 4 m-tiles); K % 128 == 0 with enough tiles -> LDS-DMA
#   256x256 / 256x128 / 128x128; otherwise register-staged 128x128 (split-K when tiles are few);
#   K % 16 != 0 or unaligned -> generic.
ACC_SHAPES = [
    (1, 64, 64), (1, 1000, 784), (3, 4096, 512), (16, 256, 4096), (17, 100, 256),
    (32, 48, 1024), (33, 160, 640), (64, 10, 256), (64, 256, 784), (65, 130, 96),
    (128, 4096, 2048), (100, 4096, 1024), (128, 2048, 2048), (300, 520, 1040), (200, 300, 16),
    (5, 7, 13), (33, 40, 30),
    (1, 1, 1), (7, 9, 0),
]


@pytest.mark.parametrize("M,N,K", ACC_SHAPES)
def test_int32_accumulator_exact(gpu, M, N, K):
    rng = np.random.default_rng(M * 7919 + N * 31 + K)
    A = _codes(rng, (M, K), -128, 127)
    B = _codes(rng, (N, K), -128, 127)
    print(f"gemm acc M={M} N={N} K={K}", flush=True)
    C = run_gemm(gpu, A, B)
    np.testing.assert_array_equal(C, O.gemm_acc(A, B))


def test_int32_accumulator_staged_many_tiles(gpu):
    """Many tiles with K % 128 != 0 (register-staged path) and ragged M, N and K."""
    rng = np.random.default_rng(5)
    M, N, K = 2000, 6400, 400
    A = _codes(rng, (M, K))
    B = _codes(rng, (N, K))
    C = run_gemm(gpu, A, B)
    np.testing.assert_array_equal(C, O.gemm_acc(A, B))


@pytest.mark.parametrize("M,N,K", [(1500, 2900, 256), (2000, 6400, 384), (257, 16384, 128),
                                   (4096, 4100, 128), (1000, 2100, 256), (300, 7000, 128),
                                   (3900, 8000, 128), (1000, 2100, 1024), (1024, 2048, 2048), (512, 4096, 1024),
                                   (500, 4000, 256)])
def test_int32_accumulator_dma_path(gpu, M, N, K):
    """The LDS-DMA 256x256, 256x128, 128x128 and 128x64 paths (K % 128 == 0, >= 128 / 256 tiles;
    one round of 128x128 tiles with a three-stage ring, half a round as 128x64 tiles) with ragged
    M and N: rows past M or N come in as zeros through the buffer bounds and are never stored."""
    rng = np.random.default_rng(M + N + K)
    A = _codes(rng, (M, K), -128, 127)
    B = _codes(rng, (N, K), -128, 127)
    print(f"gemm dma acc M={M} N={N} K={K}", flush=True)
    C = run_gemm(gpu, A, B)
    from lucid_amd import _C

    want = {(1000, 2100, 256): "gemm dma 128x128 3-stage", (1000, 2100, 1024): "gemm dma 128x128 3-stage",
            (1024, 2048, 2048): "gemm dma 128x64", (1500, 2900, 256): "gemm dma 128x128",
            (512, 4096, 1024): "gemm dma 128x64", (500, 4000, 256): "gemm dma 128x64"}
    if (M, N, K) in want:
        assert _C.last_path() == want[M, N, K]
    np.testing.assert_array_equal(C, O.gemm_acc(A, B))


@pytest.mark.parametrize("M,N,K", [(600, 8200, 128), (1000, 2100, 1024), (500, 4000, 256)])
@pytest.mark.parametrize("kind", KINDS)
def test_epilogue_kinds_dma_path(gpu, kind, M, N, K):
    """Every output kind through the LDS-staged epilogue of the DMA path (ragged N; the second
    shape is one round of 128x128 tiles with a three-stage ring, ragged M too)."""
    rng = np.random.default_rng(1000 + kind)
    A = _codes(rng, (M, K), -128, 127)
    B = _codes(rng, (N, K), -127, 127)
    a_scale = rng.uniform(1e-3, 1e-1, M).astype(np.float32)
    b_scale = rng.uniform(1e-3, 1e-1, N).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    qmin, qmax = GRID.get(kind, (-128, 127))
    out_scale, out_zp = 0.37, (128.0 if qmin == 0 else -3.0)
    zb = rng.integers(-3, 4, N).astype(np.float32)
    for za, zbv, with_bias, relu in ((None, None, True, False), (-5.0, zb, False, True)):
        acc = O.gemm_acc(A, B, 0 if za is None else int(za), None if zbv is None else zbv.astype(np.int32))
        got = run_gemm(gpu, A, B, kind, a_scale, b_scale, za, zbv, None,
                       bias if with_bias else None, out_scale, out_zp, qmin, qmax, relu)
        want = O.gemm_epilogue(acc, a_scale, b_scale, bias if with_bias else None, out_scale,
                               out_zp, qmin, qmax, kind, relu)
        if kind == O.OUT_F16:
            np.testing.assert_array_equal(got.view(np.uint16), want.view(np.uint16))
        else:
            np.testing.assert_array_equal(got.view(np.uint8), want.view(np.uint8))


@pytest.mark.parametrize("N,K", [(4096, 4096), (100, 96), (17, 80), (1000, 784), (11008, 128)])
def test_packed_weight_layout(gpu, N, K):
    rng = np.random.default_rng(N + K)
    B = _codes(rng, (N, K), -128, 127)
    np.testing.assert_array_equal(pack_weights(gpu, B).numpy()[: packed_layout_oracle(B).size],
                                  packed_layout_oracle(B))


@pytest.mark.parametrize("M,N,K", [(1, 4096, 4096), (16, 4096, 4096), (8, 11008, 4096), (1, 4096, 11008),
                                   (17, 1000, 784), (32, 100, 96), (64, 256, 784), (3, 17, 80),
                                   (100, 300, 256), (128, 4096, 4096)])
def test_packed_skinny_exact(gpu, M, N, K):
    rng = np.random.default_rng(M + N + K)
    A = _codes(rng, (M, K), -128, 127)
    B = _codes(rng, (N, K), -127, 127)
    np.testing.assert_array_equal(run_gemm(gpu, A, B, packed=True), O.gemm_acc(A, B))
    a_scale = rng.uniform(1e-3, 1e-1, M).astype(np.float32)
    b_scale = rng.uniform(1e-3, 1e-1, N).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    sums = B.astype(np.int64).sum(axis=1).astype(np.int32)
    for kind in KINDS:
        qmin, qmax = GRID.get(kind, (-128, 127))
        got = run_gemm(gpu, A, B, kind, a_scale, b_scale, za=-7.0, b_sums=sums, bias=bias,
                       out_scale=0.37, out_zp=(128.0 if qmin == 0 else 3.0), qmin=qmin, qmax=qmax,
                       relu=True, packed=True)
        want = O.gemm_w8a8(A, B, a_scale, b_scale, za=-7.0, bias=bias, out_scale=0.37,
                           out_zp=(128.0 if qmin == 0 else 3.0), qmin=qmin, qmax=qmax,
                           out_kind=kind, relu=True)
        if kind == O.OUT_F16:
            np.testing.assert_array_equal(got.view(np.uint16), want.view(np.uint16))
        else:
            np.testing.assert_array_equal(got.view(np.uint8), want.view(np.uint8))


def test_packed_rejects_large_m(gpu):
    from lucid_amd import _C

    rng = np.random.default_rng(2)
    with pytest.raises(_C.LucidError, match="M > 128"):
        run_gemm(gpu, _codes(rng, (129, 64)), _codes(rng, (16, 64)), packed=True)


def test_leading_dimensions(gpu):
    rng = np.random.default_rng(9)
    for (M, N, K) in ((8, 70, 256), (100, 200, 512), (600, 900, 256)):
        A = _codes(rng, (M, K))
        B = _codes(rng, (N, K))
        C = run_gemm(gpu, A, B, lda=K + 32, ldb=K + 48, ldc=N + 4)
        np.testing.assert_array_equal(C, O.gemm_acc(A, B))
        C = run_gemm(gpu, A, B, lda=K + 3, ldc=N + 1)  # unaligned rows -> generic path
        np.testing.assert_array_equal(C, O.gemm_acc(A, B))




@pytest.mark.parametrize("M,N,K", [(8, 200, 512), (96, 200, 512), (7, 9, 20), (300, 1000, 256)])
@pytest.mark.parametrize("kind", KINDS)
def test_epilogue_kinds_exact(gpu, M, N, K, kind):
    rng = np.random.default_rng(M + N + K + kind)
    # activations on an unsigned grid kept as (c - 128) int8 with za' = za - 128
    A = _codes(rng, (M, K), -128, 127)
    B = _codes(rng, (N, K), -127, 127)
    a_scale = rng.uniform(1e-3, 1e-1, M).astype(np.float32)
    b_scale = rng.uniform(1e-3, 1e-1, N).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    qmin, qmax = GRID.get(kind, (-128, 127))
    for za, zb, with_bias, relu in ((None, None, True, False), (-5.0, None, True, True),
                                    (3.0, rng.integers(-4, 5, N).astype(np.float32), False, True),
                                    (None, rng.integers(-2, 3, N).astype(np.float32), True, False)):
        out_scale, out_zp = 0.37, (128.0 if qmin == 0 else -3.0)
        got = run_gemm(gpu, A, B, kind, a_scale, b_scale, za, zb, None,
                       bias if with_bias else None, out_scale, out_zp, qmin, qmax, relu)
        want = O.gemm_w8a8(A, B, a_scale, b_scale, za=0.0 if za is None else za, zb=zb,
                           bias=bias if with_bias else None, out_scale=out_scale, out_zp=out_zp,
                           qmin=qmin, qmax=qmax, out_kind=kind, relu=relu)
        if kind == O.OUT_F16:
            np.testing.assert_array_equal(got.view(np.uint16), want.view(np.uint16))
        else:
            np.testing.assert_array_equal(got.view(np.uint8), want.view(np.uint8))


def test_cached_weight_sums_and_scalar_scales(gpu):
    """A caller-supplied sum_k B[n,k] (as a module caches it) and per-tensor scales."""
    rng = np.random.default_rng(3)
    M, N, K = 64, 256, 784
    A = _codes(rng, (M, K))
    B = _codes(rng, (N, K))
    sums = B.astype(np.int64).sum(axis=1).astype(np.int32)
    got = run_gemm(gpu, A, B, O.OUT_F32, np.float32(0.02), np.float32(0.03), za=7.0, b_sums=sums)
    want = O.gemm_w8a8(A, B, np.float32(0.02), np.float32(0.03), za=7.0, out_kind=O.OUT_F32)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    # the library's own row sums
    from lucid_amd import _C

    dB = _dev(gpu, B)
    out = gpu.empty((N,), np.int32, "gpu")
    _C.call("lq_row_sums_i8", dB.data_ptr(), K, N, K, out.data_ptr(), None)
    np.testing.assert_array_equal(out.numpy(), sums)


@pytest.mark.parametrize("M,N,K,packed", [(8, 200, 512, False), (8, 200, 512, True),
                                            (100, 300, 256, True), (96, 200, 512, False),
                                            (300, 1000, 256, False), (7, 9, 20, False),
                                            (512, 1024, 1024, False)])
def test_unsigned_activation_flag(gpu, M, N, K, packed):
    """LQ_EPI_A_U8S8: A holds unsigned codes u as u - 128 and the zero point passed is the
    unsigned grid's own; the kernel's result equals the signed form with za - 128."""
    from lucid_amd import _C

    rng = np.random.default_rng(M * 7 + N + K)
    U = rng.integers(0, 256, size=(M, K))
    A = (U - 128).astype(np.int8)
    B = _codes(rng, (N, K))
    b_scale = rng.uniform(1e-3, 1e-1, N).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    for zu, kind, relu in ((131.0, O.OUT_F32, False), (None, O.OUT_F32, True),
                           (0.0, O.OUT_QU8S8, True), (255.0, O.OUT_F16, False)):
        qmin, qmax = GRID.get(kind, (-128, 127))
        sums = B.astype(np.int64).sum(axis=1).astype(np.int32) if packed else None
        got = run_gemm(gpu, A, B, kind, np.float32(0.011), b_scale, zu, None, sums, bias, 0.05,
                       128.0, qmin, qmax, relu, packed=packed, flags=_C.EPI_A_U8S8)
        want = O.gemm_w8a8(A, B, np.float32(0.011), b_scale, za=(zu or 0.0) - 128.0, bias=bias,
                           out_scale=0.05, out_zp=128.0, qmin=qmin, qmax=qmax, out_kind=kind,
                           relu=relu)
        np.testing.assert_array_equal(got.view(np.uint8), want.view(np.uint8))


def test_zero_point_needs_workspace(gpu):
    from lucid_amd import _C

    rng = np.random.default_rng(1)
    A = _codes(rng, (4, 64))
    B = _codes(rng, (8, 64))
    with pytest.raises(_C.LucidError, match="workspace"):
        run_gemm(gpu, A, B, O.OUT_F32, 1.0, 1.0, za=3.0, workspace=False)


@pytest.mark.parametrize("M,N,K", [(4096, 4096, 4096), (4096, 11008, 4096), (4096, 4096, 11008),
                                   (1024, 4096, 4096), (128, 4096, 4096), (16, 11008, 4096)])
def test_baseline_sizes_checksums(gpu, M, N, K):
    rng = np.random.default_rng(M + N + K)
    A = _codes(rng, (M, K))
    B = _codes(rng, (N, K))
    print(f"gemm checksum M={M} N={N} K={K}", flush=True)
    C = run_gemm(gpu, A, B).astype(np.int64)
    A64, B64 = A.astype(np.int64), B.astype(np.int64)
    np.testing.assert_array_equal(C.sum(axis=1), A64 @ B64.sum(axis=0))
    np.testing.assert_array_equal(C.sum(axis=0), B64 @ A64.sum(axis=0))
    rows = rng.choice(M, min(M, 24), replace=False)
    np.testing.assert_array_equal(C[rows], A64[rows] @ B64.T)


@pytest.mark.parametrize("M,N,K", [(17, 70, 272), (32, 4096, 4096), (33, 4100, 4096), (64, 1000, 784),
                                   (65, 1000, 1040), (100, 300, 256), (128, 4096, 4096), (128, 11008, 4096),
                                   (96, 512, 11008)])
def test_packed_decode_split_k_exact(gpu, M, N, K):
    """33 <= M <= 128 with the packed weight and a workspace: the split-K decode kernel (A's
    K-slice staged in LDS, per-split int32 partials, ordered reduction + epilogue) -- ragged
    N, K not a multiple of 64, several splits -- bit-exact for the int32 sums and the
    requantized codes, with and without an activation zero point; M <= 32 stays on the
    skinny kernel."""
    from lucid_amd import _C

    rng = np.random.default_rng(M * 3 + N + K)
    A = _codes(rng, (M, K), -128, 127)
    B = _codes(rng, (N, K))
    C = run_gemm(gpu, A, B, packed=True)
    assert _C.last_path().startswith("gemm packed decode" if M >= 33 else "gemm packed skinny")
    np.testing.assert_array_equal(C, O.gemm_acc(A, B))
    a_scale = rng.uniform(1e-3, 1e-1, M).astype(np.float32)
    b_scale = rng.uniform(1e-3, 1e-1, N).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    sums = B.astype(np.int64).sum(axis=1).astype(np.int32)
    for za, kind in ((None, O.OUT_Q8), (-7.0, O.OUT_QU8S8), (3.0, O.OUT_F16)):
        qmin, qmax = GRID.get(kind, (-128, 127))
        got = run_gemm(gpu, A, B, kind, a_scale, b_scale, za=za, b_sums=sums if za is not None else None,
                       bias=bias, out_scale=0.37, out_zp=(128.0 if qmin == 0 else 3.0), qmin=qmin,
                       qmax=qmax, relu=True, packed=True)
        want = O.gemm_w8a8(A, B, a_scale, b_scale, za=0.0 if za is None else za, bias=bias,
                           out_scale=0.37, out_zp=(128.0 if qmin == 0 else 3.0), qmin=qmin, qmax=qmax,
                           out_kind=kind, relu=True)
        if kind == O.OUT_F16:
            np.testing.assert_array_equal(got.view(np.uint16), want.view(np.uint16))
        else:
            np.testing.assert_array_equal(got.view(np.uint8), want.view(np.uint8))


@pytest.mark.parametrize("M,N,K,packed", [(8, 2048, 512, True), (3, 100, 784, True), (512, 2048, 512, False),
                                          (70, 300, 256, False), (4096, 1024, 512, False)])
def test_gemm_gelu_epilogue_equals_gelu_kernel(gpu, M, N, K, packed):
    """LQ_EPI_GELU: the float32 output with the tanh GELU applied in the epilogue is bit for bit
    lq_gelu_tanh_f32 on the output without it (the FFN's up projection followed by F.gelu), on
    the decode (packed) and the tiled paths, with the activation zero point of the dynamic
    Linear (unsigned codes as c - 128)."""
    from lucid_amd import _C

    rng = np.random.default_rng(M + N + K)
    A = rng.integers(-128, 128, (M, K)).astype(np.int8)
    B = rng.integers(-127, 128, (N, K)).astype(np.int8)
    sa = np.float32(rng.uniform(1e-3, 1e-2))
    sb = rng.uniform(1e-4, 1e-3, N).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    sums = B.astype(np.int64).sum(1).astype(np.int32)
    kw = dict(a_scale=sa, b_scale=sb, za=131.0, b_sums=sums, bias=bias, packed=packed, flags=_C.EPI_A_U8S8)
    plain = run_gemm(gpu, A, B, O.OUT_F32, **kw)
    kw["flags"] |= _C.EPI_GELU
    fused = run_gemm(gpu, A, B, O.OUT_F32, **kw)
    dy = _dev(gpu, plain)
    g = gpu.empty(plain.shape, np.float32, "gpu")
    _C.call("lq_gelu_tanh_f32", dy.data_ptr(), g.data_ptr(), plain.size, None)
    np.testing.assert_array_equal(fused.view(np.uint32), g.numpy().view(np.uint32))
    assert_close_f32_gelu = np.max(np.abs(fused - O.gelu_tanh(plain))) <= 1e-5 * max(np.max(np.abs(plain)), 1.0)
    assert assert_close_f32_gelu


def test_gemm_gelu_rejects(gpu):
    from lucid_amd import _C

    A = np.zeros((4, 64), np.int8)
    B = np.zeros((8, 64), np.int8)
    with pytest.raises(_C.LucidError, match="GELU"):
        run_gemm(gpu, A, B, O.OUT_Q8, out_scale=1.0, flags=_C.EPI_GELU)
    with pytest.raises(_C.LucidError, match="GELU"):
        run_gemm(gpu, A, B, O.OUT_F32, relu=True, flags=_C.EPI_GELU)


# ------------------------------------------- product followed by a dynamic input step


@pytest.mark.parametrize("M,N,K,gelu,want", [
    (4096, 2048, 512, True, "gemm dma with extrema + dynamic quantize"),
    (4096, 4096, 256, False, "gemm dma with extrema + dynamic quantize"),
    (3000, 1000, 384, True, "gemm dma with extrema + dynamic quantize"),
    (500, 4000, 256, False, "gemm dma with extrema + dynamic quantize"),
    (100, 512, 512, False, "dynamic quantize two-launch"),
    (4096, 8192, 256, False, "dynamic quantize two-launch"),
    (512, 1024, 192, True, "dynamic quantize two-launch"),
])
def test_gemm_dynamic_quantize_equals_calls(gpu, M, N, K, gelu, want):
    """lq_gemm_w8a8_dynamic_quantize: the float32 product (unsigned activation codes stored as
    c - 128, bias, GELU) and the next Linear's input step -- codes and {min, max, scale, zero
    point} -- bit for bit those of lq_gemm_w8a8 followed by lq_dynamic_quantize_f32.  The DMA
    kernels fold the extrema in their epilogue (256x128, 256x256 and ragged 128x128 tiles,
    whose rows and columns past the edge must not count); a skinny M, more than 1024 tiles and
    K % 128 != 0 take the separate calls."""
    from lucid_amd import _C

    print(f"gemm dynamic quantize M={M} N={N} K={K} gelu={gelu}", flush=True)
    rng = np.random.default_rng(M + N + K)
    A = rng.integers(-128, 128, (M, K)).astype(np.int8)
    B = rng.integers(-127, 128, (N, K)).astype(np.int8)
    dA, dB = gpu.tensor(A, device="gpu"), gpu.tensor(B, device="gpu")
    sa = gpu.tensor(np.array([0.02], np.float32), device="gpu")
    za = gpu.tensor(np.array([131.0], np.float32), device="gpu")
    sb = gpu.tensor(rng.uniform(1e-3, 1e-2, N).astype(np.float32), device="gpu")
    bias = gpu.tensor(rng.standard_normal(N).astype(np.float32), device="gpu")
    sums = gpu.tensor(B.astype(np.int32).sum(axis=1).astype(np.int32), device="gpu")
    flags = _C.EPI_A_U8S8 | (_C.EPI_GELU if gelu else 0)
    eps = np.float32(1e-8)
    y1, y2 = gpu.empty((M, N), np.float32, "gpu"), gpu.empty((M, N), np.float32, "gpu")
    c1, c2 = gpu.empty((M * N,), np.int8, "gpu"), gpu.empty((M * N,), np.int8, "gpu")
    p1, p2 = gpu.empty((4,), np.float32, "gpu"), gpu.empty((4,), np.float32, "gpu")
    g_n = max(_C.lib().lq_gemm_w8a8_workspace_size(M, N, K), 16)
    gws = gpu.empty((g_n,), np.uint8, "gpu")
    _C.call("lq_gemm_w8a8", dA.data_ptr(), K, dB.data_ptr(), K, y1.data_ptr(), N, M, N, K, sa.data_ptr(), 0,
            sb.data_ptr(), 1, za.data_ptr(), None, sums.data_ptr(), bias.data_ptr(), None, None, 0, 0, _C.OUT_F32,
            flags, gws.data_ptr(), g_n, None)
    d_n = max(_C.lib().lq_dynamic_quantize_workspace_size(M * N), 16)
    dws = gpu.empty((d_n,), np.uint8, "gpu")
    _C.call("lq_dynamic_quantize_f32", y1.data_ptr(), M * N, _C.U8S8, 0, 255, eps, p1.data_ptr(), c1.data_ptr(),
            dws.data_ptr(), d_n, None)
    w_n = _C.lib().lq_gemm_w8a8_dynamic_quantize_workspace_size(M, N, K)
    ws = gpu.empty((w_n,), np.uint8, "gpu")
    _C.call("lq_gemm_w8a8_dynamic_quantize", dA.data_ptr(), K, dB.data_ptr(), K, y2.data_ptr(), M, N, K,
            sa.data_ptr(), 0, sb.data_ptr(), 1, za.data_ptr(), None, sums.data_ptr(), bias.data_ptr(), flags,
            _C.U8S8, 0, 255, eps, p2.data_ptr(), c2.data_ptr(), ws.data_ptr(), w_n, None)
    assert _C.last_path() == want  # the separate calls end with lq_dynamic_quantize_f32's own path
    np.testing.assert_array_equal(y1.numpy().view(np.uint32), y2.numpy().view(np.uint32))
    np.testing.assert_array_equal(c1.numpy(), c2.numpy())
    np.testing.assert_array_equal(p1.numpy().view(np.uint32), p2.numpy().view(np.uint32))
    yv = y2.numpy()
    np.testing.assert_array_equal(p2.numpy()[:2], np.array([yv.min(), yv.max()], np.float32))

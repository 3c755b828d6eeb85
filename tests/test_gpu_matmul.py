"""The gfx950 integer GEMM against the oracle (QuantMatMul / IntegerGemm parity).

Bar: int32 block sums and fp32 outputs bit-exact — the kernel applies the reference's
serial per-block epilogue, so nothing is left to tolerance."""
import numpy as np
import pytest

import helpers as H

pytestmark = pytest.mark.gpu

TYPES = [2, 3, 6, 7, 8]


@pytest.fixture(scope="module")
def lib(shs, oracle):
    return shs


def _w(oracle, qt, rows, cols, seed):
    return H.quantized_normal(oracle, qt, rows, cols, seed)


def test_single_gemm_config_q4_0_9216x3072_t512_is_bit_exact(lib, oracle):
    """Q4_0 W[9216×3072] ~ N(0, 0.02), X[512×3072] ~ N(0, 1): the single-GEMM workload."""
    rng = np.random.default_rng(1)
    w = oracle.quantize(2, (0.02 * rng.standard_normal((9216, 3072))).astype(np.float32))
    x = rng.standard_normal((512, 3072)).astype(np.float32)
    m = lib.WeightMatrix(2, 9216, 3072, w)
    y = m.forward(x)
    ref = oracle.matmul(2, w, 9216, 3072, x, 512)
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("T", [128, 512])
@pytest.mark.parametrize("qt", [2, 6, 7])
def test_the_seven_projections_of_a_layer_are_bit_exact(lib, oracle, qt, T):
    """q 3072→4096, k/v 3072→1024, o 4096→3072, gate/up 3072→9216, down 9216→3072, with
    weights ~ N(0, 0.02) and activations ~ N(0, 1). T = 512 is the seven-projection
    workload; the token count also selects the kernel's token-tile instantiation."""
    shapes = [(4096, 3072), (1024, 3072), (1024, 3072), (3072, 4096), (9216, 3072), (9216, 3072), (3072, 9216)]
    rng = np.random.default_rng(qt + T)
    for i, (rows, cols) in enumerate(shapes):
        w = _w(oracle, qt, rows, cols, seed=100 * qt + i)
        x = rng.standard_normal((T, cols)).astype(np.float32)
        y = lib.WeightMatrix(qt, rows, cols, w).forward(x)
        ref = oracle.matmul(qt, w, rows, cols, x, T)
        assert np.array_equal(y.view(np.uint32), ref.view(np.uint32)), (qt, rows, cols)


@pytest.mark.parametrize("qt", TYPES)
def test_block_sums_are_bit_exact(lib, oracle, qt):
    rows, cols, T = 96, 512, 45
    w = H.random_blocks(qt, rows, cols, seed=qt)
    x = np.random.default_rng(qt).standard_normal((T, cols)).astype(np.float32)
    got = lib.WeightMatrix(qt, rows, cols, w).block_sums(x)
    q, d, s = oracle.quantize_activations(x)
    assert np.array_equal(got, oracle.block_sums(qt, w, rows, cols, q, T))


@pytest.mark.parametrize("qt", TYPES)
@pytest.mark.parametrize("semantics", [0, 1])
def test_ragged_shapes_and_both_quantization_semantics(lib, oracle, qt, semantics):
    """100 rows (a partial 32-row tile), 45 tokens (a partial 32-token tile)."""
    rows, cols, T = 100, 3072, 45
    w = H.random_blocks(qt, rows, cols, seed=7 + qt)
    x = (np.random.default_rng(8).random((T, cols)) * 2 - 1).astype(np.float32)
    y = lib.WeightMatrix(qt, rows, cols, w).forward(x, semantics=semantics)
    ref = oracle.matmul(qt, w, rows, cols, x, T, semantics=semantics)
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("qt", TYPES)
def test_a_tokens_result_does_not_depend_on_the_batch(lib, oracle, qt):
    """MatMulTilingTests.ATokensResultDoesNotDependOnTheBatchItIsIn."""
    rows, cols, T = 100, 256, 13
    w = H.random_blocks(qt, rows, cols, seed=3)
    x = (np.random.default_rng(4).random((T, cols)) * 2 - 1).astype(np.float32)
    m = lib.WeightMatrix(qt, rows, cols, w)
    together = m.forward(x)
    for t in range(T):
        assert np.array_equal(m.forward(x[t:t + 1])[0], together[t])
    assert np.array_equal(m.forward(x[5:]), together[5:])
    big = np.concatenate([x] * 10)  # 130 tokens: several token tiles per wave
    assert np.array_equal(m.forward(big)[:T], together)


@pytest.mark.parametrize("qt", TYPES)
def test_decode_widths_are_bit_exact(lib, oracle, qt):
    """1-4 tokens take the weight-streaming narrow kernel: bit-exact against the oracle and
    against the same tokens inside a wide batch, with a partial row tile, an odd block
    count (7), the down projection's 288 blocks and the row counts that take 16-row (from
    16384 rows) and 32-row (from 65536, the vocabulary head) work-groups. The serial chain
    reads its operands in rounds of 16 blocks, alternating two register sets: 96 and 288
    blocks are an even number of rounds, 48 an odd one, 81 an odd one plus a remainder, 7 no
    full round."""
    rng = np.random.default_rng(20 + qt)
    for rows, cols in [(100, 3072), (64, 224), (40, 9216), (20001, 256), (65601, 256), (50, 1536), (24, 2592)]:
        w = H.random_blocks(qt, rows, cols, seed=rows + cols + qt)
        m = lib.WeightMatrix(qt, rows, cols, w)
        x = (rng.random((40, cols)) * 2 - 1).astype(np.float32)
        wide = m.forward(x)
        for T in (1, 2, 3, 4):
            y = m.forward(x[:T])
            ref = oracle.matmul(qt, w, rows, cols, x[:T], T)
            assert np.array_equal(y.view(np.uint32), ref.view(np.uint32)), (rows, cols, T)
            assert np.array_equal(y, wide[:T]), (rows, cols, T)


@pytest.mark.parametrize("qt", TYPES)
def test_a_row_subset_is_bit_identical_to_the_full_product(lib, oracle, qt):
    """MatMulTilingTests.ARowSubsetIsBitIdenticalToTheFullProduct."""
    rows, cols, T = 100, 256, 5
    ids = np.array([99, 0, 57, 57, 8, 7, 64, 63, 98], np.int32)
    w = H.random_blocks(qt, rows, cols, seed=5)
    x = (np.random.default_rng(6).random((T, cols)) * 2 - 1).astype(np.float32)
    m = lib.WeightMatrix(qt, rows, cols, w)
    full = m.forward(x)
    assert np.array_equal(m.forward_rows(ids, x), full[:, ids])


def test_a_row_subset_rejects_ids_outside_the_matrix(lib, oracle):
    w = H.random_blocks(2, 100, 256, seed=1)
    m = lib.WeightMatrix(2, 100, 256, w)
    with pytest.raises(lib.ArgumentOutOfRangeError):
        m.forward_rows([0, 100], np.zeros((1, 256), np.float32))


def test_device_pointer_entry_matches_host_entry(lib, oracle):
    """Activations already in HBM (allocated with the HIP runtime the library uses)."""
    import ctypes as C
    hip = C.CDLL("libamdhip64.so.7")
    rows, cols, T = 256, 1024, 70
    w = H.random_blocks(2, rows, cols, seed=9)
    x = np.random.default_rng(9).standard_normal((T, cols)).astype(np.float32)
    m = lib.WeightMatrix(2, rows, cols, w)
    xd, yd = C.c_void_p(), C.c_void_p()
    assert hip.hipMalloc(C.byref(xd), C.c_size_t(x.nbytes)) == 0
    assert hip.hipMalloc(C.byref(yd), C.c_size_t(T * rows * 4)) == 0
    try:
        assert hip.hipMemcpy(xd, x.ctypes.data_as(C.c_void_p), C.c_size_t(x.nbytes), 1) == 0
        m.forward_device(xd.value, T, yd.value)
        y = np.empty((T, rows), np.float32)
        assert hip.hipMemcpy(y.ctypes.data_as(C.c_void_p), yd, C.c_size_t(y.nbytes), 2) == 0
    finally:
        hip.hipFree(xd)
        hip.hipFree(yd)
    assert np.array_equal(y, m.forward(x))


def _same_bits_or_both_nan(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    nan = np.isnan(a)
    return bool(np.array_equal(nan, np.isnan(b)) and np.array_equal(a[~nan].view(np.uint32), b[~nan].view(np.uint32)))


def _edge_activations(T, cols, seed, with_saturating_blocks):
    """N(0, 1) token rows with edge blocks planted at random (token, block) slots: all
    zero; exact ties (max 127, so d = inv = 1 and ±2.5, 0.5, 1.5, 126.5 are ties); d
    subnormal with a finite inverse (max 1e-36); very large maxima (1e30, 3e38); and, when
    asked, the blocks whose values convert to 0x80000000 and saturate to code −128: maxima
    whose 1/d overflows (1e-37, 1e-40) and one infinite element."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((T, cols)).astype(np.float32)
    tie = np.zeros(32, np.float32)
    tie[:8] = [127.0, 2.5, -2.5, 3.5, 0.5, -0.5, 1.5, -126.5]
    kinds = ["zero", "tie", 1e-36, 1e30, 3e38] + (["inf", 1e-37, 1e-40] if with_saturating_blocks else [])
    B = cols // 32
    for n, kind in enumerate(kinds * 6):
        t, b = int(rng.integers(T)), int(rng.integers(B))
        blk = x[t, 32 * b:32 * b + 32]
        if kind == "zero":
            blk[:] = 0
        elif kind == "tie":
            blk[:] = rng.permutation(tie) * (1 if n % 2 else -1)
        elif kind == "inf":
            blk[int(rng.integers(32))] = np.inf * (1 if n % 2 else -1)
        else:
            blk[:] = (blk / np.abs(blk).max() * kind).astype(np.float32)
    return x


@pytest.mark.parametrize("qt", TYPES)
@pytest.mark.parametrize("semantics", [0, 1])
def test_activation_edge_blocks_are_bit_exact(lib, oracle, qt, semantics):
    """The quantizer's edges (IntegerDotTests.cs:128-173, IntegerGemm.cs:89-95) through the
    whole GEMM at 100 rows × 3072 × 45 tokens (partial row and token tiles), and through
    the decode-width kernel for the first 4 tokens. Outputs that overflow to ±inf or NaN
    (an infinite element, or a 3e38 max times a weight scale) are compared as NaN = NaN
    (the NaN payload is the hardware's). For Q8_0 the saturating blocks are left out: its
    kernel multiplies the signed bytes, so its zero-point correction comes from the
    saturated codes, where IntegerGemm's comes from the wrapped int32 block sum (a known
    divergence, only for blocks holding a non-finite value or a max below 3.7e-37)."""
    rows, cols, T = 100, 3072, 45
    w = H.random_blocks(qt, rows, cols, seed=70 + qt)
    x = _edge_activations(T, cols, seed=qt + 10 * semantics, with_saturating_blocks=qt != 8)
    m = lib.WeightMatrix(qt, rows, cols, w)
    with np.errstate(all="ignore"):
        ref = oracle.matmul(qt, w, rows, cols, x, T, semantics=semantics)
    y = m.forward(x, semantics=semantics)
    assert _same_bits_or_both_nan(y, ref)
    if semantics == 0:
        assert _same_bits_or_both_nan(m.forward(x[:4]), ref[:4])
        assert _same_bits_or_both_nan(m.forward(x[3:4]), ref[3:4])


@pytest.mark.parametrize("qt", [2, 3, 6, 7])
def test_block_sums_at_the_activation_edges(lib, oracle, qt):
    """The exact int32 block sums −z·Σa + Σ u·a for the edge blocks, against the oracle fed
    the quantizer's own block sums (wrapped, as IntegerGemm's int32 vector adds wrap)."""
    rows, cols, T = 64, 1024, 33
    w = H.random_blocks(qt, rows, cols, seed=90 + qt)
    x = _edge_activations(T, cols, seed=5, with_saturating_blocks=True)
    with np.errstate(all="ignore"):
        q, d, s = oracle.quantize_activations(x)
    got = lib.WeightMatrix(qt, rows, cols, w).block_sums(x)
    assert np.array_equal(got, oracle.block_sums(qt, w, rows, cols, q, T, s))


@pytest.mark.parametrize("qt", [6, 7])
def test_q5_blocks_with_every_fifth_bit_set_at_t512(lib, oracle, qt):
    """Q5_0/Q5_1 weights whose 32 high bits are all set (u = 16..31), mixed with random
    blocks, at 512 tokens, 100 rows (a partial row tile) and 500 tokens (a partial token tile)."""
    rows, cols = 100, 3072
    w = H.random_blocks(qt, rows, cols, seed=qt).reshape(-1, H.TYPE_SIZE[qt]).copy()
    qh = 2 if qt == 6 else 4
    rng = np.random.default_rng(qt)
    pick = rng.random(w.shape[0]) < 0.5
    w[pick, qh:qh + 4] = 0xFF
    w = w.reshape(-1)
    m = lib.WeightMatrix(qt, rows, cols, w)
    for T in (512, 500):
        x = rng.standard_normal((T, cols)).astype(np.float32)
        y = m.forward(x)
        ref = oracle.matmul(qt, w, rows, cols, x, T)
        assert np.array_equal(y.view(np.uint32), ref.view(np.uint32)), T


# With unit block scales (helpers.unit_scale_weights / unit_scale_activations) the GEMM's
# outputs are exact sums of its int32 block sums.
@pytest.mark.parametrize("qt", TYPES)
def test_hot_gemm_single_block_outputs_are_the_int32_block_sums(lib, oracle, qt):
    """K = 32: every output of the production GEMM (k_gemm, the same instantiations the model
    runs) is one block's integer sum Σ w·q, against int64 brute force."""
    rng = np.random.default_rng(70 + qt)
    rows, cols, T = 256, 32, 96
    w, v = H.unit_scale_weights(oracle, qt, rows, cols, rng)
    x = H.unit_scale_activations(T, cols, rng)
    y = lib.WeightMatrix(qt, rows, cols, w).forward(x)
    ref = x.astype(np.int64) @ v.astype(np.int64).T
    assert np.array_equal(y.astype(np.int64), ref) and np.all(y == ref)


@pytest.mark.parametrize("qt,rows,cols,T", [
    (2, 9216, 3072, 512),   # two token tiles per work-group, 2-block stages (the gate|up instantiation)
    (2, 3072, 4096, 1024),  # one token tile, 4-block stages in a 3-slot ring (o and down)
    (2, 256, 416, 64),      # 13 blocks: an odd last stage
    (6, 256, 416, 512),
    (7, 3072, 1024, 512),
    (3, 1024, 2048, 128),
    (8, 1024, 2048, 128),
])
def test_hot_gemm_unit_scale_outputs_are_exact_sums_of_block_sums(lib, oracle, qt, rows, cols, T):
    """The whole K loop with unit scales: y = Σ_b I_b exactly, against float64 brute force
    (exact: every product and partial sum is an integer far below 2^53). The precondition
    Σ|w|·|q| < 2^24 keeps every partial sum of the fp32 chain exact."""
    rng = np.random.default_rng(rows + cols + T + qt)
    w, v = H.unit_scale_weights(oracle, qt, rows, cols, rng)
    x = H.unit_scale_activations(T, cols, rng)
    bound = np.abs(x).astype(np.float64) @ np.abs(v).astype(np.float64).T
    assert bound.max() < 2 ** 24
    y = lib.WeightMatrix(qt, rows, cols, w).forward(x)
    ref = x.astype(np.float64) @ v.astype(np.float64).T
    assert np.array_equal(y.astype(np.float64), ref)

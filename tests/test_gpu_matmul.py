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


@pytest.mark.parametrize("qt", [2, 6, 7])
def test_the_seven_projections_of_a_layer_are_bit_exact(lib, oracle, qt):
    """q 3072→4096, k/v 3072→1024, o 4096→3072, gate/up 3072→9216, down 9216→3072."""
    shapes = [(4096, 3072), (1024, 3072), (1024, 3072), (3072, 4096), (9216, 3072), (9216, 3072), (3072, 9216)]
    rng = np.random.default_rng(qt)
    T = 128
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

"""Pins the CPU oracle (oracle/) before it is trusted as the GPU path's checker.

Each test checks the oracle against something that does not restate it: the
reference's golden vectors (tests/golden/quantization_legacy.json, from llm-shield's
tests/fixtures/quantization.json), a replay of the generator that produced them,
numpy/float64 closed forms, exact rational arithmetic, and invariants the reference's
own tests assert (IntegerDotTests, MatMulTilingTests, KernelTests, RopeAndCacheTests).
"""
import base64
import json
import math
from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest

import helpers as H
import np_reference as NR

GOLDEN = Path(__file__).resolve().parent / "golden" / "quantization_legacy.json"
LEGACY = ("Q4_0", "Q4_1", "Q5_0", "Q5_1", "Q8_0")


@pytest.fixture(scope="module")
def fixture_cases():
    return {c["type"]: c for c in json.loads(GOLDEN.read_text())["cases"]}


# ----------------------------------------------------------- block formats

@pytest.mark.parametrize("name", LEGACY)
def test_dequantize_matches_gguf_fixture_bit_exactly(oracle, fixture_cases, name):
    """DequantizerParityTests.Dequantize_MatchesReference, tightened from 1e-4 to bit-exact."""
    case = fixture_cases[name]
    qt = oracle.TYPE_NAMES[name]
    assert case["block_size"] == 32 and case["type_size"] == oracle.TYPE_SIZE[qt]
    for kind in ("quantized", "synthetic"):
        raw = base64.b64decode(case[kind]["bytes"])
        exp = np.array(case[kind]["expected"], np.float32)
        got = oracle.dequantize(qt, raw, exp.size)
        assert np.array_equal(got.view(np.uint32), exp.view(np.uint32)), (name, kind)


def test_quantizer_replays_the_fixture_generator(oracle, fixture_cases):
    """Replays gen_quant_fixtures.py's numpy draw order (seed 20260806): our ggml quantizer
    must reproduce the `quantized` blobs byte for byte, and the acceptance loop of the
    synthetic blobs (finite, |v| ≤ 1e6) must land on exactly the fixture's blocks."""
    rng = np.random.default_rng(20260806)
    for _ in range(3):  # F32, F16, BF16 entries draw 64 normals each
        rng.standard_normal(64).astype(np.float32)
    for name in LEGACY:
        qt = oracle.TYPE_NAMES[name]
        ts = oracle.TYPE_SIZE[qt]
        src = rng.standard_normal(8 * 32).astype(np.float32) * 0.35
        mine = oracle.quantize(qt, src).tobytes()
        assert mine == base64.b64decode(fixture_cases[name]["quantized"]["bytes"]), name
        kept = []
        for _ in range(200):
            if len(kept) >= 8:
                break
            raw = rng.integers(0, 256, size=ts, dtype=np.uint8)
            vals = oracle.dequantize(qt, raw.tobytes(), 32)
            if not np.all(np.isfinite(vals)) or np.max(np.abs(vals)) > 1e6:
                continue
            kept.append(raw.tobytes())
        assert b"".join(kept) == base64.b64decode(fixture_cases[name]["synthetic"]["bytes"]), name


def test_decode_agrees_with_independent_numpy_decoder(oracle):
    for qt in (2, 3, 6, 7, 8):
        raw = H.random_blocks(qt, 5, 128, seed=qt)
        a = oracle.dequantize(qt, raw, 5 * 128).astype(np.float64)
        b = NR.dequantize(qt, raw, 5, 128).reshape(-1)
        assert np.allclose(a, b, rtol=1e-6, atol=1e-7), qt


def test_half_to_float_is_exact_for_every_bit_pattern(oracle):
    """MatMulTilingTests.TheVectorisedHalfConversionIsExactForEveryBitPattern."""
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    lib = oracle.lib()
    got = np.array([lib.ora_half_to_float(int(b)) for b in bits], np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_float_to_half_rounds_like_numpy(oracle):
    rng = np.random.default_rng(7)
    x = np.concatenate([rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-9, 5, 20000),
                        np.array([65504, 65519.9, 65520, 6.1e-5, 5.96e-8, 2.98e-8, 1e-9, -0.0, 0.0], np.float32)])
    lib = oracle.lib()
    got = np.array([lib.ora_float_to_half(float(v)) for v in x], np.uint16)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


# --------------------------------------------------- activation quantization

def test_activation_quantization_round_trips_within_half_a_step(oracle):
    """IntegerDotTests.ActivationQuantizationRoundTripsWithinOnePercent, both semantics."""
    rng = np.random.default_rng(11)
    x = (rng.random(1024) * 8 - 4).astype(np.float32)
    for sem in (0, 1):
        q, d, s = oracle.quantize_activations(x, sem)
        back = q.reshape(-1, 32).astype(np.float64) * d[:, None]
        bmax = np.abs(x.reshape(-1, 32)).max(axis=1, keepdims=True)
        worst = np.max(np.abs(back - x.reshape(-1, 32)) / bmax)
        assert worst < 1.0 / 254 * 1.05, (sem, worst)
        assert np.array_equal(s, q.reshape(-1, 32).astype(np.int64).sum(axis=1))


def test_activation_quantization_handles_an_all_zero_block(oracle):
    for sem in (0, 1):
        q, d, s = oracle.quantize_activations(np.zeros(64, np.float32), sem)
        assert not q.any() and not d.any() and not s.any()


def test_activation_quantization_tie_rounding(oracle):
    """max = 127 gives d = 1 and inv = 1 exactly, so x·inv = ±2.5 is an exact tie:
    IntegerGemm rounds to even (vcvtps2dq), IntegerDot away from zero."""
    x = np.zeros(32, np.float32)
    x[0], x[1], x[2], x[3] = 127.0, 2.5, -2.5, 3.5
    q0, d0, _ = oracle.quantize_activations(x, 0)
    q1, d1, _ = oracle.quantize_activations(x, 1)
    assert d0[0] == 1.0 and d1[0] == 1.0
    assert list(q0[:4]) == [127, 2, -2, 4]
    assert list(q1[:4]) == [127, 3, -3, 4]


def test_activation_quantization_matches_numpy_float32(oracle):
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((16, 3072)) * rng.random((16, 1)) * 5).astype(np.float32)
    q, d, s = oracle.quantize_activations(x)
    qn, dn, sn = NR.quantize_acts(x)
    assert np.array_equal(q.reshape(16, -1, 32), qn) and np.array_equal(d.reshape(16, -1), dn)
    assert np.array_equal(s.reshape(16, -1), sn)


def edge_blocks():
    """Activation blocks at the quantizer's edges, one per 32-value block: all zero; exact
    ties; a max that makes d subnormal with a finite inverse (1e-36); a max whose d is so
    small that 1/d overflows to +inf (1e-37 and 1e-40); very large maxima (1e30, 3e38);
    one infinite element; ordinary N(0, 1)."""
    rng = np.random.default_rng(77)
    blocks = [np.zeros(32)]
    tie = np.zeros(32)
    tie[:8] = [127.0, 2.5, -2.5, 3.5, 0.5, -0.5, 1.5, -126.5]
    blocks.append(tie)
    for mx in (1e-36, 1e-37, 1e-40, 1e30, 3e38):
        b = rng.standard_normal(32)
        blocks.append(b / np.abs(b).max() * mx)
    inf = rng.standard_normal(32)
    inf[5] = np.inf
    blocks.append(inf)
    blocks.append(rng.standard_normal(32))
    return np.concatenate(blocks).astype(np.float32)


def test_activation_quantization_at_the_edges_follows_the_x86_conversion(oracle):
    """IntegerGemm.QuantizeActivations converts with vcvtps2dq, packs with signed
    saturation and sums the unsaturated int32 values (IntegerGemm.cs:110-136). numpy's
    float32 → int32 cast on this x86 host is the same conversion (NaN and out-of-range
    give 0x80000000), so it restates the edges independently: a block whose 1/d
    overflows converts every value to 0x80000000 (code −128, sum 32·2^31 ≡ 0 mod 2^32),
    and an infinite element makes d infinite, inverse 0 and that value NaN."""
    x = edge_blocks()
    q, d, s = oracle.quantize_activations(x, 0)
    xb = x.reshape(-1, 32)
    mx = np.max(np.abs(xb), axis=1)
    dn = (mx / np.float32(127)).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        inv = np.where(dn != 0, np.float32(1) / dn, np.float32(0)).astype(np.float32)
        v = np.rint((xb * inv[:, None]).astype(np.float32))
        q32 = v.astype(np.int32)
    assert np.array_equal(d, dn)
    assert np.array_equal(q.reshape(-1, 32), np.clip(q32, -128, 127).astype(np.int8))
    assert np.array_equal(s, (q32.astype(np.int64).sum(axis=1) % 2 ** 32).astype(np.uint32).view(np.int32))
    assert np.isinf(inv[3]) and np.all(q32[3] == np.iinfo(np.int32).min) and s[3] == 0
    assert list(q[32:40]) == [127, 2, -2, 4, 0, 0, 2, -126]
    assert 0 < d[2] < np.finfo(np.float32).tiny and np.isfinite(inv[2]) and np.abs(q32[2]).max() == 127
    assert q32[7, 5] == np.iinfo(np.int32).min and s[7] == np.iinfo(np.int32).min


def test_dot_semantics_at_the_edges(oracle):
    """IntegerDot rounds half away from zero, converts as .NET 9+ does (saturating, NaN to
    0) and clamps to ±127; its scale is stored as fp16, so a block max below ≈3.8e-6 keeps
    d = 0 while its codes still come from the float inverse."""
    x = edge_blocks()
    q, d, s = oracle.quantize_activations(x, 1)
    assert list(q[32:40]) == [127, 3, -3, 4, 1, -1, 2, -127]
    assert np.all(q.reshape(-1, 32)[3] == np.where(x.reshape(-1, 32)[3] > 0, 127, -127))
    assert d[2] == 0 and d[3] == 0 and q.reshape(-1, 32)[7, 5] == 0
    assert np.array_equal(s, q.reshape(-1, 32).astype(np.int64).sum(axis=1))


def test_block_sums_follow_the_zero_point_form_at_the_edges(oracle):
    """I = −z·Σa + Σ u·a in int32 (IntegerGemm.cs:384-397), from the quantizer's block sum,
    brute-forced in int64 and wrapped; for the saturated blocks this differs from
    Σ (u − z)·codes."""
    x = edge_blocks()
    q, d, s = oracle.quantize_activations(x, 0)
    T, cols = 1, x.size
    for qt in (2, 3, 6, 7, 8):
        w = H.random_blocks(qt, 3, cols, seed=qt)
        got = oracle.block_sums(qt, w, 3, cols, q, T, s)
        wi, _, _ = NR.decode_blocks(qt, w, 3, cols)
        z = {2: 8, 3: 0, 6: 16, 7: 0, 8: 128}[qt]
        u = wi.reshape(3, -1, 32) + z
        qq = q.reshape(-1, 32).astype(np.int64)
        ref = np.einsum("rbk,bk->rb", u, qq) - z * s.astype(np.int64)[None, :]
        ref = (ref % 2 ** 32).astype(np.uint32).view(np.int32)
        assert np.array_equal(got[0], ref), qt


def test_dot_semantics_scale_is_fp16_rounded(oracle):
    x = np.random.default_rng(4).standard_normal(3072).astype(np.float32)
    _, d0, _ = oracle.quantize_activations(x, 0)
    _, d1, _ = oracle.quantize_activations(x, 1)
    assert np.array_equal(d1, d0.astype(np.float16).astype(np.float32))


# -------------------------------------------------------------------- GEMM

@pytest.mark.parametrize("qt", [2, 3, 6, 7, 8])
def test_block_sums_equal_numpy_int64_brute_force(oracle, qt):
    rows, cols, T = 40, 256, 7
    w = H.random_blocks(qt, rows, cols, seed=10 + qt)
    x = np.random.default_rng(qt).standard_normal((T, cols)).astype(np.float32)
    q, d, s = oracle.quantize_activations(x)
    got = oracle.block_sums(qt, w, rows, cols, q, T)
    wi, _, _ = NR.decode_blocks(qt, w, rows, cols)
    ref = np.einsum("rbk,tbk->trb", wi.reshape(rows, -1, 32), q.reshape(T, -1, 32).astype(np.int64))
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("qt", [2, 3, 6, 7, 8])
def test_matmul_matches_float64_closed_form(oracle, qt):
    rows, cols, T = 64, 3072, 5
    w = H.random_blocks(qt, rows, cols, seed=20 + qt)
    x = np.random.default_rng(30 + qt).standard_normal((T, cols)).astype(np.float32)
    y = oracle.matmul(qt, w, rows, cols, x, T)
    ref = NR.qmatmul(qt, w, rows, cols, x)
    assert H.rel_l2(y, ref) < 1e-6
    assert H.max_close(y, ref) < 1e-5


def _rn32(fr: Fraction) -> Fraction:
    """Exact round-to-nearest-even of a rational to binary32 (normal/subnormal range)."""
    if fr == 0:
        return Fraction(0)
    sign = -1 if fr < 0 else 1
    x = abs(fr)
    e = x.numerator.bit_length() - x.denominator.bit_length()
    if Fraction(2) ** e > x:
        e -= 1
    e = max(e, -126)
    ulp = Fraction(2) ** (e - 23)
    m = x / ulp
    n = m.numerator // m.denominator
    rem = m - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    return sign * n * ulp


@pytest.mark.parametrize("qt", [2, 3, 6, 7, 8])
def test_matmul_epilogue_is_the_reference_fma_chain_bit_exactly(oracle, qt):
    """acc = fma(float(I_b), RN(d_w·d_a), acc) block by block, then fma(m_w, RN(d_a·Σq), acc)
    (IntegerGemm.cs:399-412), evaluated in exact rational arithmetic."""
    rows, cols, T = 6, 128, 3
    w = H.random_blocks(qt, rows, cols, seed=40 + qt)
    x = np.random.default_rng(50 + qt).standard_normal((T, cols)).astype(np.float32)
    y = oracle.matmul(qt, w, rows, cols, x, T)
    wi, dw, mw = NR.decode_blocks(qt, w, rows, cols)
    q, da, s = NR.quantize_acts(x)
    B = cols // 32
    for t in range(T):
        for r in range(rows):
            acc = Fraction(0)
            for b in range(B):
                I = int(np.dot(wi[r, 32 * b:32 * b + 32], q[t, b]))
                sc = _rn32(Fraction(float(dw[r, b])) * Fraction(float(da[t, b])))
                acc = _rn32(Fraction(I) * sc + acc)
                if qt in (3, 7):
                    ds = _rn32(Fraction(float(da[t, b])) * Fraction(int(s[t, b])))
                    acc = _rn32(Fraction(float(mw[r, b])) * ds + acc)
            assert np.float32(float(acc)) == y[t, r], (t, r)


@pytest.mark.parametrize("qt", [2, 3, 6, 7, 8])
def test_integer_path_agrees_with_float_path(oracle, qt):
    """IntegerDotTests.IntegerPathAgreesWithFloatPath: relative L2 < 1e-2 at T ∈ {3, 13}.
    The normalised-bias bound (< 2e-3) is evaluated over 64 tokens: for the offset types
    the m·(d_a·Σq − Σx) term shares each token's quantization error across all rows, so
    over 3 tokens the statistic is noise of order 2e-3 for any random draw, while a
    missing or misplaced offset shifts it by orders of magnitude more."""
    rows, cols = 100, 3072
    w = H.random_blocks(qt, rows, cols, seed=21)
    for T in (3, 13, 64):
        x = (np.random.default_rng(5).random((T, cols)) * 2 - 1).astype(np.float32)
        yi = oracle.matmul(qt, w, rows, cols, x, T).astype(np.float64)
        yf = x.astype(np.float64) @ NR.dequantize(qt, w, rows, cols).T
        rel = np.sqrt(np.sum((yi - yf) ** 2) / np.sum(yf ** 2))
        assert rel < 1e-2, (T, rel)
        if T == 64:
            bias = np.mean(yi - yf) / np.sqrt(np.mean(yf ** 2))
            assert abs(bias) < 2e-3, bias


@pytest.mark.parametrize("qt", [2, 3, 6, 7, 8])
def test_a_tokens_result_does_not_depend_on_the_batch(oracle, qt):
    """MatMulTilingTests.ATokensResultDoesNotDependOnTheBatchItIsIn (bit-exact)."""
    rows, cols, T = 100, 256, 13
    w = H.random_blocks(qt, rows, cols, seed=3)
    x = (np.random.default_rng(4).random((T, cols)) * 2 - 1).astype(np.float32)
    together = oracle.matmul(qt, w, rows, cols, x, T)
    for t in range(T):
        assert np.array_equal(oracle.matmul(qt, w, rows, cols, x[t:t + 1], 1)[0], together[t])
    assert np.array_equal(oracle.matmul(qt, w, rows, cols, x[5:], 8), together[5:])


@pytest.mark.parametrize("qt", [2, 3, 6, 7, 8])
def test_a_row_subset_is_bit_identical_to_the_full_product(oracle, qt):
    """MatMulTilingTests.ARowSubsetIsBitIdenticalToTheFullProduct."""
    rows, cols, T = 100, 256, 5
    ids = np.array([99, 0, 57, 57, 8, 7, 64, 63, 98], np.int32)
    w = H.random_blocks(qt, rows, cols, seed=5)
    x = (np.random.default_rng(6).random((T, cols)) * 2 - 1).astype(np.float32)
    full = oracle.matmul(qt, w, rows, cols, x, T)
    sub = oracle.matmul(qt, w, rows, cols, x, T, row_ids=ids)
    assert np.array_equal(sub, full[:, ids])


def test_a_row_subset_rejects_ids_outside_the_matrix(oracle):
    w = H.random_blocks(2, 100, 256, seed=1)
    with pytest.raises(IndexError):
        oracle.matmul(2, w, 100, 256, np.zeros((1, 256), np.float32), 1, row_ids=[0, 100])


def test_gather_rows_rejects_out_of_range_ids(oracle):
    w = H.random_blocks(2, 10, 64, seed=1)
    with pytest.raises(IndexError):
        oracle.gather_rows(2, w, 10, 64, [3, 10])


# ------------------------------------------------------------- elementwise

def test_rmsnorm_matches_closed_form(oracle):
    rng = np.random.default_rng(1)
    for n in (1, 7, 16, 33, 3072, 9216):
        x = rng.standard_normal(n).astype(np.float32) * 3
        w = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
        y = oracle.rmsnorm(x, w, 1e-5)
        ref = NR.rmsnorm(x, w, 1e-5)
        assert np.max(np.abs(y - ref) / np.maximum(1, np.abs(ref))) < 1e-5, n


def test_softmax_properties(oracle):
    """KernelTests: sums to one, shift invariant, survives logits of 50/95/400, a fully
    masked row becomes uniform."""
    rng = np.random.default_rng(2)
    x = rng.standard_normal(37).astype(np.float32)
    p = oracle.softmax(x)
    assert abs(float(p.astype(np.float64).sum()) - 1) < 1e-6
    assert np.allclose(oracle.softmax(x + 100), p, rtol=1e-5, atol=1e-7)
    for big in (50.0, 95.0, 400.0):
        y = oracle.softmax(np.array([big, 0, -big, big - 1], np.float32))
        assert np.all(np.isfinite(y)) and abs(y.sum() - 1) < 1e-6
    u = oracle.softmax(np.full(5, -np.inf, np.float32))
    assert np.allclose(u, 0.2)
    ref = np.exp(x.astype(np.float64) - x.max())
    assert np.allclose(p, ref / ref.sum(), rtol=1e-5)


def test_swiglu_matches_closed_form(oracle):
    rng = np.random.default_rng(3)
    g = rng.standard_normal(9216).astype(np.float32) * 4
    u = rng.standard_normal(9216).astype(np.float32)
    y = oracle.swiglu(g, u)
    gd = g.astype(np.float64)
    ref = gd / (1 + np.exp(-gd)) * u
    assert np.max(np.abs(y - ref) / np.maximum(1, np.abs(ref))) < 1e-5


def test_dot4_and_add_scaled4_match_closed_forms(oracle):
    rng = np.random.default_rng(4)
    for n in (8, 13, 128):
        s = rng.standard_normal(n).astype(np.float32)
        a = [rng.standard_normal(n).astype(np.float32) for _ in range(4)]
        r = oracle.dot4(s, a)
        for k in range(4):
            assert abs(r[k] - float(np.dot(a[k].astype(np.float64), s))) < 1e-5 * max(1, abs(r[k]))
        w = rng.standard_normal(4).astype(np.float32)
        d = oracle.add_scaled4(s, a, w)
        for k in range(4):
            assert np.allclose(d[k], a[k] + w[k] * s.astype(np.float64), rtol=1e-6, atol=1e-6)


# ------------------------------------------------------------------- RoPE

def test_rope_identity_at_position_zero_and_norm_preserving(oracle):
    cfg = oracle.make_config()
    f, ms = oracle.rope_freqs(cfg)
    assert ms == 1.0
    x = np.random.default_rng(5).standard_normal(4 * 128).astype(np.float32)
    assert np.array_equal(oracle.rope_apply(f, ms, 128, x, 4, 128, 0), x)
    y = oracle.rope_apply(f, ms, 128, x, 4, 128, 777)
    n0 = np.hypot(x[0::2].astype(np.float64), x[1::2])
    n1 = np.hypot(y[0::2].astype(np.float64), y[1::2])
    assert np.allclose(n0, n1, rtol=1e-6)


def test_rope_rotates_adjacent_pairs(oracle):
    """RopeAndCacheTests.RotationPairsAdjacentElements: e_0 only mixes into element 1."""
    cfg = oracle.make_config()
    f, ms = oracle.rope_freqs(cfg)
    x = np.zeros(128, np.float32)
    x[0] = 1.0
    y = oracle.rope_apply(f, ms, 128, x, 1, 128, 5)
    assert abs(y[0] - math.cos(5 * f[0])) < 1e-6 and abs(y[1] - math.sin(5 * f[0])) < 1e-6
    assert not np.any(y[2:])


def test_rope_heads_are_independent_and_match_closed_form(oracle):
    cfg = oracle.make_config()
    f, ms = oracle.rope_freqs(cfg)
    assert np.allclose(f, 1.0 / 1e6 ** (np.arange(64) * 2 / 128), rtol=1e-6)
    rng = np.random.default_rng(6)
    x = rng.standard_normal(3 * 128).astype(np.float32)
    y = oracle.rope_apply(f, ms, 128, x, 3, 128, 1000)
    ref = NR.rope(x[None, :], 3, 128, [1000], 1e6, 128)[0]
    assert np.max(np.abs(y - ref)) < 1e-4
    y1 = oracle.rope_apply(f, ms, 128, x[128:256], 1, 128, 1000)
    assert np.array_equal(y1, y[128:256])


def test_yarn_magnitude_scale(oracle):
    """RopeAndCacheTests: mscale = 1 when mscale == mscale_all_dim ("apply_scale": false);
    fallback 1 + 0.1·ln(16) when mscale_all_dim is absent; ramp endpoints and monotonicity."""
    yarn = dict(rope_scale=16.0, rope_orig_ctx=16384, yarn_active=1, yarn_beta_fast=32.0, yarn_beta_slow=1.0)
    f, ms = oracle.rope_freqs(oracle.make_config(yarn_mscale=1.0, yarn_mscale_all_dim=1.0, **yarn))
    assert ms == 1.0
    _, ms2 = oracle.rope_freqs(oracle.make_config(**yarn))
    assert abs(ms2 - (1 + 0.1 * math.log(16))) < 1e-6
    ext = (1.0 / 1e6 ** (np.arange(64) * 2 / 128)).astype(np.float32)
    assert abs(f[0] - ext[0]) <= 1e-7 * ext[0]
    assert abs(f[-1] - ext[-1] / 16) <= 1e-6 * ext[-1]
    assert np.all(np.diff(f.astype(np.float64)) < 0)


# ------------------------------------------------------------------- model

TINY = dict(n_layer=2, hidden=256, n_head=4, n_kv_head=1, head_dim=128, ffn=512, vocab=512)


@pytest.fixture(scope="module")
def tiny_model(oracle):
    cfg = oracle.make_config(**TINY)
    tensors, types = H.synth_model_tensors(oracle, cfg, 2, seed=123)
    return cfg, tensors, types


def test_forward_matches_independent_numpy_model(oracle, tiny_model):
    cfg, tensors, types = tiny_model
    toks = np.random.default_rng(9).integers(0, cfg.vocab, 40)
    m = oracle.OracleModel(cfg, tensors, types, cap=64)
    got = m.forward(toks, head_mode=2)
    ref = NR.forward(cfg, tensors, types, toks)
    assert H.rel_l2(got, ref) < 2e-3, H.rel_l2(got, ref)


def test_forward_layer_outputs_match_numpy(oracle, tiny_model):
    cfg, tensors, types = tiny_model
    toks = np.random.default_rng(10).integers(0, cfg.vocab, 33)
    cap = {}
    m = oracle.OracleModel(cfg, tensors, types, cap=64)
    m.forward(toks, head_mode=0, capture=lambda n, a: cap.__setitem__(n, a))
    for l in range(cfg.n_layer):
        ref = NR.forward(cfg, tensors, types, toks, head=None, layers=l + 1)
        assert H.rel_l2(cap[f"blk.{l}.output"], ref) < 1e-3, l


def test_prefix_cache_is_bit_identical(oracle, tiny_model):
    """SystemPromptCacheTests.CachedAndUncachedProduceIdenticalLogits on the oracle."""
    cfg, tensors, types = tiny_model
    toks = np.random.default_rng(11).integers(0, cfg.vocab, 50)
    m = oracle.OracleModel(cfg, tensors, types, cap=64)
    full = m.forward(toks, head_mode=2)
    m.reset()
    m.forward(toks[:17], head_mode=0)
    snap = m.snapshot()
    m.reset()
    m.restore(snap, 17)
    cached = m.forward(toks[17:], head_mode=2)
    assert np.array_equal(full, cached)
    m.reset()
    sel = m.forward(toks, head_mode=1, vocab_ids=[5, 7, 400])
    assert np.array_equal(sel, full[[5, 7, 400]])


def test_score_closed_form(oracle):
    logits = np.array([1.0, 3.0, 2.0, -1.0, 0.5], np.float32)
    s, y, n = oracle.score(logits, 3, 2)
    assert y == 3.0 and n == 0.5
    assert abs(s - 1 / (1 + math.exp(-(3.0 - 0.5)))) < 1e-6


@pytest.mark.parametrize("qt", [2, 3, 6, 7, 8])
def test_gemm_with_unit_block_scales_is_the_integer_product(oracle, qt):
    """With every weight block at d = 1 (m = 0) and every activation block at d_a = 1, the
    epilogue multiplies each int32 block sum by RN(1·1) = 1 and adds no offset, so the GEMM is
    the integer product of the weights' and activations' values — a closed form that a wrong
    nibble order, a dropped zero point or a misplaced fifth bit would break. 13 blocks."""
    rng = np.random.default_rng(90 + qt)
    w, v = H.unit_scale_weights(oracle, qt, 96, 416, rng)
    x = H.unit_scale_activations(40, 416, rng)
    y = oracle.matmul(qt, w, 96, 416, x, 40)
    assert np.array_equal(y.astype(np.float64), x.astype(np.float64) @ v.astype(np.float64).T)

"""Shared test utilities: seeded inputs, synthetic weights, tolerance metrics."""
import numpy as np

TYPE_SIZE = {2: 18, 3: 20, 6: 22, 7: 24, 8: 34}


def rel_l2(a, e):
    a = np.asarray(a, np.float64)
    e = np.asarray(e, np.float64)
    return float(np.linalg.norm(a - e) / max(np.linalg.norm(e), 1e-30))


def max_close(a, e):
    """Numeric.Close's metric: |a−e| / max(1, |e|), worst element."""
    a = np.asarray(a, np.float64)
    e = np.asarray(e, np.float64)
    return float(np.max(np.abs(a - e) / np.maximum(1.0, np.abs(e)))) if a.size else 0.0


def random_blocks(qtype, rows, cols, seed, scale_lo=0.005, scale_hi=0.025):
    """Random payload bytes with every fp16 scale (and min) forced to a sane value
    (the construction of MatMulTilingTests.Weights / IntegerDotTests.QuantizeRows)."""
    rng = np.random.default_rng(seed)
    ts = TYPE_SIZE[qtype]
    raw = rng.integers(0, 256, size=rows * (cols // 32) * ts, dtype=np.uint8).reshape(-1, ts)
    d = (scale_lo + (scale_hi - scale_lo) * rng.random(raw.shape[0])).astype(np.float16)
    raw[:, 0:2] = d.view(np.uint8).reshape(-1, 2)
    if qtype in (3, 7):
        m = (-0.03 * rng.random(raw.shape[0])).astype(np.float16)
        raw[:, 2:4] = m.view(np.uint8).reshape(-1, 2)
    return raw.reshape(-1)


def quantized_normal(oracle, qtype, rows, cols, seed, std=0.02, mean=0.0):
    rng = np.random.default_rng(seed)
    w = (mean + std * rng.standard_normal((rows, cols))).astype(np.float32)
    return oracle.quantize(qtype, w)


def synth_model_tensors(oracle, cfg, qtype, seed, embd_type=None):
    """Host-side random-init model of cfg's shape: N(0,0.02) matrices, N(1,0.1) norms."""
    embd_type = qtype if embd_type is None else embd_type
    rng = np.random.default_rng(seed)
    tensors, types = {}, {}

    def mat(name, t, ne0, ne1):
        w = (0.02 * rng.standard_normal((ne1, ne0))).astype(np.float32)
        tensors[name] = oracle.quantize(t, w)
        types[name] = t

    def vec(name, n):
        tensors[name] = (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)
        types[name] = 0

    qd, kvd = cfg.n_head * cfg.head_dim, cfg.n_kv_head * cfg.head_dim
    mat("token_embd.weight", embd_type, cfg.hidden, cfg.vocab)
    vec("output_norm.weight", cfg.hidden)
    for l in range(cfg.n_layer):
        p = f"blk.{l}."
        vec(p + "attn_norm.weight", cfg.hidden)
        mat(p + "attn_q.weight", qtype, cfg.hidden, qd)
        mat(p + "attn_k.weight", qtype, cfg.hidden, kvd)
        mat(p + "attn_v.weight", qtype, cfg.hidden, kvd)
        mat(p + "attn_output.weight", qtype, qd, cfg.hidden)
        vec(p + "ffn_norm.weight", cfg.hidden)
        mat(p + "ffn_gate.weight", qtype, cfg.hidden, cfg.ffn)
        mat(p + "ffn_up.weight", qtype, cfg.hidden, cfg.ffn)
        mat(p + "ffn_down.weight", qtype, cfg.ffn, cfg.hidden)
    return tensors, types


def shs_config_from_oracle(shs, cfg):
    """shieldstral.ModelConfig with the oracle Config's fields."""
    return shs.ModelConfig(cfg.n_layer, cfg.hidden, cfg.n_head, cfg.n_kv_head, cfg.head_dim, cfg.ffn, cfg.vocab,
                           cfg.eps, cfg.rope_theta, cfg.rope_dim, cfg.rope_scale, cfg.rope_orig_ctx,
                           cfg.yarn_beta_fast, cfg.yarn_beta_slow, cfg.yarn_ext_factor, cfg.yarn_mscale,
                           cfg.yarn_mscale_all_dim, cfg.rope_attn_factor, cfg.attn_temperature, bool(cfg.yarn_active))


CAPTURE_NAMES_PER_LAYER = ("attn_norm", "q_rope", "k_rope", "v", "attn_weighted", "attn_out", "post_attn",
                           "ffn_norm", "ffn_out", "output")


# Unit block scales make the hot GEMM print its integer block sums: weights whose every
# block quantizes with d = 1 (and m = 0) hold integer codes, activations whose every block
# has max |x| = 127 quantize with d_a = 1 to codes equal to their values, so each scale
# RN(d_w·d_a) is 1, the offset term is 0 and the fp32 chain acc = fma(I_b, 1, acc) adds exact
# integers while |partial sums| < 2^24: y = Σ_b I_b exactly, I_b = Σ_k w_k·q_k.
UNIT_RANGE = {2: (-8, 7), 3: (0, 15), 6: (-16, 15), 7: (0, 31), 8: (-127, 127)}


def unit_scale_weights(oracle, qt, rows, cols, rng):
    lo, hi = UNIT_RANGE[qt]
    v = rng.integers(lo, hi + 1, (rows, cols)).astype(np.float32)
    blk = v.reshape(rows, cols // 32, 32)
    if qt in (2, 6):
        blk[:, :, 0] = lo            # the max-|x| element fixes d = lo / lo = 1
    elif qt in (3, 7):
        blk[:, :, 0], blk[:, :, 1] = lo, hi  # min 0 and max 2^n − 1: d = 1, m = 0
    else:
        blk[:, :, 0] = hi            # max |x| = 127: d = 1
    w = oracle.quantize(qt, v)
    assert np.array_equal(oracle.dequantize(qt, w, rows * cols).reshape(rows, cols), v)
    return w, v


def unit_scale_activations(T, cols, rng):
    x = rng.integers(-127, 128, (T, cols)).astype(np.float32)
    x.reshape(T, cols // 32, 32)[:, :, 0] = 127
    return x

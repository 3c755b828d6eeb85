"""Independent numpy restatement of the Shieldstral forward pass, used to pin the oracle.

Shares no code with oracle/: block decoding, activation quantization, attention and the
layer loop are written here from the reference's description (MinistralModel.cs:183-482,
IntegerGemm.cs, Kernels.cs, Rope.cs) in vectorized numpy. Dot products and everything
after the int8 quantization are evaluated in float64; only the quantizer itself runs in
float32, because its rounding points are what the reference computes.
"""
import numpy as np


def decode_blocks(qtype, raw, rows, cols):
    """→ (w int64 [rows, cols] signed weights u−z, d float64 [rows, B], m float64 [rows, B])."""
    B = cols // 32
    ts = {2: 18, 3: 20, 6: 22, 7: 24, 8: 34}[qtype]
    blk = np.asarray(raw, np.uint8).reshape(rows, B, ts)
    d = blk[:, :, 0:2].copy().view(np.float16).reshape(rows, B).astype(np.float64)
    m = np.zeros((rows, B))
    if qtype == 8:
        w = blk[:, :, 2:].view(np.int8).astype(np.int64)
        return w.reshape(rows, cols), d, m
    if qtype in (3, 7):
        m = blk[:, :, 2:4].copy().view(np.float16).reshape(rows, B).astype(np.float64)
    qs_off = {2: 2, 3: 4, 6: 6, 7: 8}[qtype]
    qs = blk[:, :, qs_off:qs_off + 16].astype(np.int64)
    u = np.concatenate([qs & 0x0F, qs >> 4], axis=2)  # element j low nibble, 16+j high nibble
    if qtype in (6, 7):
        qh_off = 2 if qtype == 6 else 4
        qh = blk[:, :, qh_off:qh_off + 4].copy().view("<u4").reshape(rows, B, 1).astype(np.int64)
        bits = (qh >> np.arange(32)) & 1
        u = u | (bits << 4)
    z = {2: 8, 3: 0, 6: 16, 7: 0}[qtype]
    return (u - z).reshape(rows, cols), d, m


def dequantize(qtype, raw, rows, cols):
    w, d, m = decode_blocks(qtype, raw, rows, cols)
    B = cols // 32
    return (w.reshape(rows, B, 32) * d[:, :, None] + m[:, :, None]).reshape(rows, cols)


def quantize_acts(x):
    """IntegerGemm.QuantizeActivations in float32 numpy: (q int64, d f32, s int64) per 32-block."""
    x = np.asarray(x, np.float32)
    T, K = x.shape
    xb = x.reshape(T, K // 32, 32)
    mx = np.max(np.abs(xb), axis=2)
    d = (mx / np.float32(127)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(d != 0, np.float32(1) / d, np.float32(0)).astype(np.float32)
    q = np.rint((xb * inv[:, :, None]).astype(np.float32)).astype(np.int64)
    return q, d, q.sum(axis=2)


def qmatmul(qtype, raw, rows, cols, x):
    """Σ_b d_w·d_a·I_b (+ m_w·d_a·Σq) in float64."""
    w, dw, mw = decode_blocks(qtype, raw, rows, cols)
    q, da, s = quantize_acts(x)
    B = cols // 32
    I = np.einsum("rbk,tbk->trb", w.reshape(rows, B, 32), q)
    y = np.einsum("trb,rb,tb->tr", I.astype(np.float64), dw, da.astype(np.float64))
    if qtype in (3, 7):
        y += np.einsum("rb,tb->tr", mw, da.astype(np.float64) * s)
    return y


def rmsnorm(x, g, eps):
    x = np.asarray(x, np.float64)
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * np.asarray(g, np.float64)


def rope_freqs(cfg):
    """Rotary frequencies and magnitude factor in float64 (Rope.cs:33-106): plain
    1/θ^(2i/d)/factor, or YaRN's ramp between the interpolated and extrapolated
    frequencies with ggml's correction dimensions and the mscale ratio."""
    d = cfg.rope_dim
    half = d // 2
    i = np.arange(half, dtype=np.float64)
    ext = 1.0 / cfg.rope_theta ** (2.0 * i / d)
    factor = float(cfg.rope_scale)
    if not cfg.yarn_active:
        return ext / factor, float(cfg.rope_attn_factor)
    bf, bs = float(cfg.yarn_beta_fast), float(cfg.yarn_beta_slow)

    def corr(rot):
        return d * np.log(cfg.rope_orig_ctx / (rot * 2 * np.pi)) / (2 * np.log(cfg.rope_theta))

    if bf == 0 and bs == 0:
        low, high = np.inf, half - 1.0
    else:
        low, high = max(0.0, np.floor(corr(bf))), min(half - 1.0, np.ceil(corr(bs)))
    ramp = np.clip((i - low) / max(0.001, high - low), 0.0, 1.0)
    mix = (1.0 - ramp) * cfg.yarn_ext_factor
    freqs = ext / factor * (1.0 - mix) + ext * mix

    def msc(m):
        return 1.0 if factor <= 1 else 0.1 * m * np.log(factor) + 1.0

    m = cfg.yarn_mscale if cfg.yarn_mscale != 0 else 1.0
    ratio = msc(m) / msc(cfg.yarn_mscale_all_dim) if cfg.yarn_mscale_all_dim != 0 else msc(1.0)
    return freqs, ratio * cfg.rope_attn_factor


def query_temperature(cfg, pos):
    """Llama-4 attention temperature per position (MinistralModel.cs:471-482)."""
    pos = np.asarray(pos, np.float64)
    if cfg.rope_orig_ctx <= 0 or cfg.attn_temperature == 0:
        return np.ones_like(pos)
    return 1.0 + cfg.attn_temperature * np.log1p(np.floor(pos / cfg.rope_orig_ctx))


def rope(x, heads, hd, pos, theta, rope_dim, freqs=None, mscale=1.0):
    """Adjacent-pair rotation; x [T, heads·hd]; pos [T]."""
    T = x.shape[0]
    half = rope_dim // 2
    freq = 1.0 / theta ** (2.0 * np.arange(half) / rope_dim) if freqs is None else np.asarray(freqs, np.float64)
    ang = np.asarray(pos, np.float64)[:, None] * freq[None, :]
    c, s = mscale * np.cos(ang)[:, None, :], mscale * np.sin(ang)[:, None, :]
    y = np.array(x, np.float64).reshape(T, heads, hd)
    x0, x1 = y[:, :, 0:rope_dim:2].copy(), y[:, :, 1:rope_dim:2].copy()
    y[:, :, 0:rope_dim:2] = x0 * c - x1 * s
    y[:, :, 1:rope_dim:2] = x0 * s + x1 * c
    return y.reshape(T, heads * hd)


def swiglu(g, u):
    """Kernels.SwiGlu (Kernels.cs:83-90) in float64: sigmoid(g)·(g·u)."""
    g = np.asarray(g, np.float64)
    return g * np.asarray(u, np.float64) / (1.0 + np.exp(-g))


def attention(q, k, v, n_head, n_kv, hd, q_pos, k_pos):
    """Causal GQA: query head h reads kv head h // (n_head / n_kv)."""
    T = q.shape[0]
    group = n_head // n_kv
    out = np.zeros((T, n_head * hd))
    qh = q.reshape(T, n_head, hd)
    kh = k.reshape(-1, n_kv, hd)
    vh = v.reshape(-1, n_kv, hd)
    mask = np.asarray(k_pos)[None, :] <= np.asarray(q_pos)[:, None]
    for h in range(n_head):
        g = h // group
        sc = qh[:, h, :] @ kh[:, g, :].T / np.sqrt(hd)
        sc = np.where(mask, sc, -np.inf)
        sc = sc - sc.max(axis=1, keepdims=True)
        p = np.exp(sc)
        p /= p.sum(axis=1, keepdims=True)
        out[:, h * hd:(h + 1) * hd] = p @ vh[:, g, :]
    return out


def forward(cfg, tensors, types, tokens, head="full", vocab_ids=None, layers=None):
    """Whole-prompt prefill from an empty cache; returns logits of the last position."""
    L, H, KV, hd = cfg.n_layer, cfg.n_head, cfg.n_kv_head, cfg.head_dim
    qd, kvd = H * hd, KV * hd
    toks = np.asarray(tokens)
    T = toks.size
    emb = dequantize(types["token_embd.weight"], tensors["token_embd.weight"], cfg.vocab, cfg.hidden)
    h = emb[toks].astype(np.float64)
    pos = np.arange(T)
    freqs, ms = rope_freqs(cfg)
    temp = query_temperature(cfg, pos)[:, None]
    for l in range(L if layers is None else layers):
        p = f"blk.{l}."
        x = rmsnorm(h, tensors[p + "attn_norm.weight"], cfg.eps)
        q = qmatmul(types[p + "attn_q.weight"], tensors[p + "attn_q.weight"], qd, cfg.hidden, x)
        k = qmatmul(types[p + "attn_k.weight"], tensors[p + "attn_k.weight"], kvd, cfg.hidden, x)
        v = qmatmul(types[p + "attn_v.weight"], tensors[p + "attn_v.weight"], kvd, cfg.hidden, x)
        q = rope(q, H, hd, pos, cfg.rope_theta, cfg.rope_dim, freqs, ms) * temp
        k = rope(k, KV, hd, pos, cfg.rope_theta, cfg.rope_dim, freqs, ms)
        ctx = attention(q, k, v, H, KV, hd, pos, pos)
        h = h + qmatmul(types[p + "attn_output.weight"], tensors[p + "attn_output.weight"], cfg.hidden, qd, ctx)
        x = rmsnorm(h, tensors[p + "ffn_norm.weight"], cfg.eps)
        g = qmatmul(types[p + "ffn_gate.weight"], tensors[p + "ffn_gate.weight"], cfg.ffn, cfg.hidden, x)
        u = qmatmul(types[p + "ffn_up.weight"], tensors[p + "ffn_up.weight"], cfg.ffn, cfg.hidden, x)
        a = swiglu(g, u)
        h = h + qmatmul(types[p + "ffn_down.weight"], tensors[p + "ffn_down.weight"], cfg.hidden, cfg.ffn, a)
    if head is None:
        return h
    last = rmsnorm(h[-1:], tensors["output_norm.weight"], cfg.eps)
    logits = qmatmul(types["token_embd.weight"], tensors["token_embd.weight"], cfg.vocab, cfg.hidden, last)[0]
    return logits if vocab_ids is None else logits[np.asarray(vocab_ids)]

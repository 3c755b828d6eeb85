"""Pins the oracle's layer stage by stage against the independent numpy restatement.

Every numpy stage is fed the oracle's own captured input for that stage, so an int8
code that flips in one stage cannot compound into the next: each comparison measures
one stage's arithmetic alone, and each is bound at 1e-5 relative. The head shapes cover
GQA groups of 1 to 4 query heads per KV head, including the real model's 32/8, so the
query-head → KV-head mapping (MinistralModel.cs:392, kv head = h / group) and the
per-head KV cache layout (KvCache.cs:43-60, snapshot order KvCache.cs:94-112) are both
pinned. A wrong mapping such as h % n_kv, or a wrong per-head cache stride, moves
attn_weighted by O(1).

The FFN has no capture between ffn_norm and ffn_out (the reference observes none,
MinistralModel.cs:226-231), so its pieces are pinned one at a time: the oracle's gate
and up products and its SwiGLU against numpy, then the captured ffn_out against the
oracle's own matmul of that SwiGLU output (the composition) and against numpy's.
"""
import math

import numpy as np
import pytest

import helpers as H
import np_reference as NR

STAGE_TOL = 1e-5

HEADS = [(4, 1), (4, 2), (8, 2), (8, 4), (6, 3), (32, 8)]

YARN = dict(rope_scale=16.0, rope_orig_ctx=16, yarn_active=1, yarn_beta_fast=32.0, yarn_beta_slow=1.0,
            yarn_ext_factor=1.0, yarn_mscale=1.0, yarn_mscale_all_dim=1.0, attn_temperature=0.1)


def rel(a, e):
    """Worst of the tensor's relative L2 error and its worst element's |a−e|/max(1,|e|)."""
    return max(H.rel_l2(a, e), H.max_close(a, e))


def small_config(oracle, n_head, n_kv, **kw):
    return oracle.make_config(n_layer=2, hidden=256, n_head=n_head, n_kv_head=n_kv, head_dim=128, ffn=512,
                              vocab=512, **kw)


def run_captured(oracle, cfg, tensors, types, toks, model=None, head_mode=2):
    cap = {}
    m = model or oracle.OracleModel(cfg, tensors, types, cap=128)
    logits = m.forward(toks, head_mode=head_mode, capture=lambda n, a: cap.__setitem__(n, a))
    return m, cap, logits


def check_layer_stages(oracle, cfg, tensors, types, cap, l, pos, k_all=None, v_all=None, k_pos=None):
    """Every stage of layer l, each from the oracle's captured input. k_all/v_all/k_pos
    give the full cache contents for a pass that starts after a cached prefix."""
    p = f"blk.{l}."
    hd, H_, KV = cfg.head_dim, cfg.n_head, cfg.n_kv_head
    qd, kvd = H_ * hd, KV * hd
    x_in = cap["embeddings"] if l == 0 else cap[f"blk.{l - 1}.output"]
    errs = {}

    errs["attn_norm"] = rel(cap[p + "attn_norm"], NR.rmsnorm(x_in, tensors[p + "attn_norm.weight"], cfg.eps))

    xn = cap[p + "attn_norm"]
    freqs, ms = NR.rope_freqs(cfg)
    temp = NR.query_temperature(cfg, pos)[:, None]
    q = NR.qmatmul(types[p + "attn_q.weight"], tensors[p + "attn_q.weight"], qd, cfg.hidden, xn)
    q = NR.rope(q, H_, hd, pos, cfg.rope_theta, cfg.rope_dim, freqs, ms) * temp
    errs["q_rope"] = rel(cap[p + "q_rope"], q)
    k = NR.qmatmul(types[p + "attn_k.weight"], tensors[p + "attn_k.weight"], kvd, cfg.hidden, xn)
    k = NR.rope(k, KV, hd, pos, cfg.rope_theta, cfg.rope_dim, freqs, ms)
    errs["k_rope"] = rel(cap[p + "k_rope"], k)
    v = NR.qmatmul(types[p + "attn_v.weight"], tensors[p + "attn_v.weight"], kvd, cfg.hidden, xn)
    errs["v"] = rel(cap[p + "v"], v)

    if k_all is None:
        k_all, v_all, k_pos = cap[p + "k_rope"], cap[p + "v"], pos
    ctx = NR.attention(cap[p + "q_rope"].astype(np.float64), np.asarray(k_all, np.float64),
                       np.asarray(v_all, np.float64), H_, KV, hd, pos, k_pos)
    errs["attn_weighted"] = rel(cap[p + "attn_weighted"], ctx)

    o = NR.qmatmul(types[p + "attn_output.weight"], tensors[p + "attn_output.weight"], cfg.hidden, qd,
                   cap[p + "attn_weighted"])
    errs["attn_out"] = rel(cap[p + "attn_out"], o)
    assert np.array_equal(cap[p + "post_attn"], x_in + cap[p + "attn_out"]), (l, "post_attn")

    errs["ffn_norm"] = rel(cap[p + "ffn_norm"],
                           NR.rmsnorm(cap[p + "post_attn"], tensors[p + "ffn_norm.weight"], cfg.eps))

    fn = cap[p + "ffn_norm"]
    T = fn.shape[0]
    g_o = oracle.matmul(types[p + "ffn_gate.weight"], tensors[p + "ffn_gate.weight"], cfg.ffn, cfg.hidden, fn, T)
    u_o = oracle.matmul(types[p + "ffn_up.weight"], tensors[p + "ffn_up.weight"], cfg.ffn, cfg.hidden, fn, T)
    errs["ffn_gate"] = rel(g_o, NR.qmatmul(types[p + "ffn_gate.weight"], tensors[p + "ffn_gate.weight"],
                                           cfg.ffn, cfg.hidden, fn))
    errs["ffn_up"] = rel(u_o, NR.qmatmul(types[p + "ffn_up.weight"], tensors[p + "ffn_up.weight"],
                                         cfg.ffn, cfg.hidden, fn))
    a_o = oracle.swiglu(g_o, u_o)
    errs["swiglu"] = rel(a_o, NR.swiglu(g_o, u_o))
    down_w, down_t = tensors[p + "ffn_down.weight"], types[p + "ffn_down.weight"]
    assert np.array_equal(cap[p + "ffn_out"], oracle.matmul(down_t, down_w, cfg.hidden, cfg.ffn, a_o, T)), \
        (l, "ffn_out composition")
    errs["ffn_out"] = rel(cap[p + "ffn_out"], NR.qmatmul(down_t, down_w, cfg.hidden, cfg.ffn, a_o))
    assert np.array_equal(cap[p + "output"], cap[p + "post_attn"] + cap[p + "ffn_out"]), (l, "output")

    bad = {k: e for k, e in errs.items() if not e <= STAGE_TOL}
    assert not bad, (l, bad)
    return errs


@pytest.mark.parametrize("n_head,n_kv", HEADS)
def test_every_stage_matches_numpy(oracle, n_head, n_kv):
    cfg = small_config(oracle, n_head, n_kv)
    tensors, types = H.synth_model_tensors(oracle, cfg, 2, seed=100 + n_head * 10 + n_kv)
    toks = np.random.default_rng(n_head + n_kv).integers(0, cfg.vocab, 40)
    m, cap, logits = run_captured(oracle, cfg, tensors, types, toks)
    pos = np.arange(toks.size)
    for l in range(cfg.n_layer):
        check_layer_stages(oracle, cfg, tensors, types, cap, l, pos)

    # KvCache.Snapshot order: keys [layer][kv head][pos][dim], then values, each equal to
    # the rows the layer stored.
    hd, T = cfg.head_dim, toks.size
    snap = m.snapshot()
    per = cfg.n_layer * n_kv * T * hd
    ks = snap[:per].reshape(cfg.n_layer, n_kv, T, hd)
    vs = snap[per:].reshape(cfg.n_layer, n_kv, T, hd)
    for l in range(cfg.n_layer):
        assert np.array_equal(ks[l].transpose(1, 0, 2).reshape(T, n_kv * hd), cap[f"blk.{l}.k_rope"])
        assert np.array_equal(vs[l].transpose(1, 0, 2).reshape(T, n_kv * hd), cap[f"blk.{l}.v"])

    last = cap[f"blk.{cfg.n_layer - 1}.output"][-1:]
    assert rel(cap["final_norm"], NR.rmsnorm(last, tensors["output_norm.weight"], cfg.eps)) <= STAGE_TOL
    ref = NR.qmatmul(types["token_embd.weight"], tensors["token_embd.weight"], cfg.vocab, cfg.hidden,
                     cap["final_norm"])[0]
    assert rel(logits, ref) <= STAGE_TOL
    emb = NR.dequantize(types["token_embd.weight"], tensors["token_embd.weight"], cfg.vocab, cfg.hidden)
    assert np.array_equal(cap["embeddings"], emb[toks].astype(np.float32))


@pytest.mark.parametrize("n_head,n_kv", [(4, 2), (8, 2)])
def test_stages_after_a_cached_prefix(oracle, n_head, n_kv):
    """A pass that appends at position 17 attends to the restored prefix: its queries sit
    at positions 17.., its keys are the snapshot's rows followed by its own."""
    cfg = small_config(oracle, n_head, n_kv)
    tensors, types = H.synth_model_tensors(oracle, cfg, 2, seed=7 + n_head)
    toks = np.random.default_rng(3).integers(0, cfg.vocab, 41)
    m = oracle.OracleModel(cfg, tensors, types, cap=128)
    m.forward(toks[:17], head_mode=0)
    snap = m.snapshot()
    m.reset()
    m.restore(snap, 17)
    _, cap, _ = run_captured(oracle, cfg, tensors, types, toks[17:], model=m)
    hd, P = cfg.head_dim, 17
    per = cfg.n_layer * n_kv * P * hd
    ks = snap[:per].reshape(cfg.n_layer, n_kv, P, hd)
    vs = snap[per:].reshape(cfg.n_layer, n_kv, P, hd)
    pos = np.arange(P, toks.size)
    for l in range(cfg.n_layer):
        k_all = np.concatenate([ks[l].transpose(1, 0, 2).reshape(P, n_kv * hd), cap[f"blk.{l}.k_rope"]])
        v_all = np.concatenate([vs[l].transpose(1, 0, 2).reshape(P, n_kv * hd), cap[f"blk.{l}.v"]])
        check_layer_stages(oracle, cfg, tensors, types, cap, l, pos, k_all, v_all, np.arange(toks.size))


def test_stages_with_yarn_and_the_query_temperature(oracle):
    """The real checkpoint's RoPE (YaRN keys as the converter writes them,
    tools/convert_shieldstral_to_gguf.py:307-319) with a 16-token original context, so
    the Llama-4 query temperature engages from position 16 inside a 40-token prompt."""
    cfg = small_config(oracle, 8, 2, **YARN)
    freqs, ms = oracle.rope_freqs(cfg)
    f64, ms64 = NR.rope_freqs(cfg)
    assert ms == ms64 == 1.0
    assert np.max(np.abs(freqs - f64) / f64) < 1e-6
    tensors, types = H.synth_model_tensors(oracle, cfg, 2, seed=31)
    toks = np.random.default_rng(4).integers(0, cfg.vocab, 40)
    _, cap, _ = run_captured(oracle, cfg, tensors, types, toks)
    pos = np.arange(toks.size)
    assert NR.query_temperature(cfg, pos)[-1] == pytest.approx(1 + 0.1 * math.log(3))
    for l in range(cfg.n_layer):
        check_layer_stages(oracle, cfg, tensors, types, cap, l, pos)


def test_yarn_frequencies_and_mscale_match_numpy(oracle):
    """Rope.cs:33-106 for several factor / context / beta settings, mscale ≠ 1 included."""
    cases = [dict(rope_scale=16.0, rope_orig_ctx=16384, yarn_mscale=1.0, yarn_mscale_all_dim=1.0),
             dict(rope_scale=16.0, rope_orig_ctx=16384),
             dict(rope_scale=4.0, rope_orig_ctx=4096, yarn_mscale=0.707, yarn_mscale_all_dim=1.0),
             dict(rope_scale=8.0, rope_orig_ctx=2048, yarn_beta_fast=0.0, yarn_beta_slow=0.0),
             dict(rope_scale=2.0, rope_orig_ctx=8192, yarn_ext_factor=0.5, rope_attn_factor=1.25)]
    for kw in cases:
        base = dict(yarn_active=1, yarn_beta_fast=32.0, yarn_beta_slow=1.0)
        base.update(kw)
        cfg = oracle.make_config(**base)
        f, ms = oracle.rope_freqs(cfg)
        f64, ms64 = NR.rope_freqs(cfg)
        assert np.max(np.abs(f - f64) / f64) < 2e-6, kw
        assert abs(ms - ms64) < 1e-6 * ms64, kw


def test_expf_is_within_one_ulp_of_float64_exp(oracle):
    """ora_expf against float64 exp on every 257th float32 in (−104, 89] (8.7·10⁶
    arguments). An exhaustive sweep of all 2.24·10⁹ floats in that range measured a
    worst error of 0.99999997 ulp under the same metric; the test bounds it at < 1 ulp.
    The ulp is the smaller of the float32 spacings either side of the true value."""
    pats = np.arange(0, 2 ** 32, 257, dtype=np.uint64).astype(np.uint32)
    x = pats.view(np.float32)
    x = x[np.isfinite(x) & (x > np.float32(-104.0)) & (x <= np.float32(89.0))]
    y = oracle.expf(x)
    e = np.exp(x.astype(np.float64))
    keep = e < float(np.finfo(np.float32).max)
    assert np.all(np.isinf(y[~keep]))
    y, e = y[keep].astype(np.float64), e[keep]
    ef = e.astype(np.float32)
    lo = np.nextafter(ef, np.float32(0))
    sp = np.minimum(np.spacing(np.abs(ef)), np.where(lo == 0, np.spacing(np.abs(ef)), np.spacing(np.abs(lo))))
    sp = np.maximum(sp.astype(np.float64), 2.0 ** -149)
    err = np.abs(y - e) / sp
    assert err.max() < 1.0, (float(err.max()), float(x[keep][np.argmax(err)]))


def test_expf_edges(oracle):
    big = np.float32(float.fromhex("0x1.62e42ep+6"))  # largest float whose exp is finite
    x = np.array([0.0, -0.0, big, np.nextafter(big, np.float32(np.inf)), 89.0, np.inf, -np.inf, np.nan,
                  -104.0, -100.0, -87.0, 1.0, -1.0], np.float32)
    y = oracle.expf(x)
    assert y[0] == 1.0 and y[1] == 1.0
    assert np.isfinite(y[2]) and abs(float(y[2]) / math.exp(float(big)) - 1) < 2 ** -23
    assert np.isinf(y[3]) and np.isinf(y[4]) and np.isinf(y[5])
    assert y[6] == 0.0 and np.isnan(y[7]) and y[8] == 0.0
    assert 0 < y[9] < 2.0 ** -126 and abs(float(y[9]) - math.exp(-100.0)) <= 2.0 ** -149  # subnormal
    assert abs(float(y[10]) / math.exp(-87.0) - 1) < 2 ** -23
    assert abs(float(y[11]) - math.e) <= 2 ** -22 and abs(float(y[12]) - math.exp(-1)) <= 2 ** -24

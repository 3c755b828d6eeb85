"""The HIP forward pass (MinistralModel / ShieldstralModerator parity) against the oracle.

Bar: bit-exact. Every stage performs the reference's floating-point operations in the
reference's order (RMSNorm's lane sums, the int8 quantization, the serial GEMM epilogue,
RoPE from the same cos/sin, attention's Dot4 chains / softmax / AddScaled4 chain, the
deterministic exp both sides share), so every captured tensor, the KV cache and the
logits must match the oracle bit for bit. The Score is then identical too; the looser
bounds kept below (1e-4) are the north-star tolerances, asserted as well."""
import math
import os
import tempfile

import numpy as np
import pytest

import helpers as H

pytestmark = pytest.mark.gpu

TINY = dict(n_layer=2, hidden=256, n_head=4, n_kv_head=1, head_dim=128, ffn=512, vocab=512)
FP_TOL = 1e-4


@pytest.fixture(scope="module")
def tiny(shs, oracle):
    cfg = oracle.make_config(**TINY)
    tensors, types = H.synth_model_tensors(oracle, cfg, 2, seed=7)
    gpu = shs.MinistralModel.from_tensors(H.shs_config_from_oracle(shs, cfg), tensors, types)
    ora = oracle.OracleModel(cfg, tensors, types, cap=600)
    return cfg, tensors, types, gpu, ora


def test_forward_matches_oracle_and_first_layer_is_bit_exact(shs, oracle, tiny):
    cfg, tensors, types, gpu, ora = tiny
    toks = np.random.default_rng(1).integers(0, cfg.vocab, 77)
    gcap, ocap = {}, {}
    gpu.reset_kv_cache()
    gpu.set_capture(lambda n, a: gcap.__setitem__(n, a))
    try:
        g = gpu.forward(toks)
    finally:
        gpu.set_capture(None)
    ora.reset()
    o = ora.forward(toks, head_mode=2, capture=lambda n, a: ocap.__setitem__(n, a))
    expected = {"embeddings", "final_norm", "logits"} | {
        f"blk.{l}.{s}" for l in range(cfg.n_layer) for s in H.CAPTURE_NAMES_PER_LAYER}
    assert set(gcap) == expected == set(ocap)
    for name in sorted(expected):
        assert np.array_equal(gcap[name], ocap[name]), (name, H.rel_l2(gcap[name], ocap[name]))
    assert np.array_equal(g, o)


def test_both_attention_paths_match_the_oracle(shs, oracle, tiny):
    """A 32-query item runs scores, softmax and values in one kernel (k_attn_fused), its
    first score tiles in the block's LDS (35 tiles of 32 keys beside the row maxima, the row
    sums and the 16 KB of query rows in 160 KB) and any later ones in the item's scratch
    region; items past 256 key tiles take the three-kernel path. A pass of 1110 keys fills the
    LDS exactly (35 tiles, the last partial), ones of 1300 and 3100 spill their later items'
    tiles past the 35th, and one of 8300 runs both kernels in each layer (its last items,
    past 8192 keys, through the three). All bit-exact, including a pass that starts mid-tile."""
    cfg, tensors, types, gpu, ora = tiny
    long_ora = oracle.OracleModel(cfg, tensors, types, cap=8400)
    rng = np.random.default_rng(11)
    ids = [1, 200, 511]
    for prefix, n, fused in ((0, 70, True), (45, 50, True), (0, 1110, True), (0, 1300, True), (0, 3100, True),
                             (0, 8300, False)):
        toks = rng.integers(0, cfg.vocab, prefix + n)
        gpu.reset_kv_cache()
        long_ora.reset()
        if prefix:
            gpu.prefill(toks[:prefix])
            long_ora.forward(toks[:prefix], head_mode=0)
        gpu.profile(True)
        gpu.profile_reset()
        try:
            g = gpu.forward_selected(toks[prefix:], ids)
            n_fused = gpu.profile_read("k_attn_fused")[0]
            n_split = gpu.profile_read("k_attn_softmax")[0]
        finally:
            gpu.profile(False)
        o = long_ora.forward(toks[prefix:], head_mode=1, vocab_ids=ids)
        assert np.array_equal(g, o), (prefix, n, H.rel_l2(g, o))
        assert (n_fused, n_split) == ((cfg.n_layer, 0) if fused else (cfg.n_layer, cfg.n_layer)), (prefix, n)


def test_attention_with_two_query_heads_per_kv_head(shs, oracle):
    """GQA groups below 4: the score kernel leaves a block's extra waves idle and the fused
    kernel skips the missing heads' blocks; the attention stays bit-exact (40-, 1100-, 1300-
    and 3100-token passes take the fused kernel, the last two spilling tiles past the 35th;
    an 8300-token one also the three-kernel path)."""
    cfg = oracle.make_config(n_layer=1, hidden=256, n_head=4, n_kv_head=2, head_dim=128, ffn=512, vocab=512)
    tensors, types = H.synth_model_tensors(oracle, cfg, 2, seed=13)
    gpu = shs.MinistralModel.from_tensors(H.shs_config_from_oracle(shs, cfg), tensors, types)
    ora = oracle.OracleModel(cfg, tensors, types, cap=8400)
    rng = np.random.default_rng(17)
    ids = [0, 77, 300]
    try:
        for n in (40, 1100, 1300, 3100, 8300):
            toks = rng.integers(0, cfg.vocab, n)
            gpu.reset_kv_cache()
            ora.reset()
            g = gpu.forward_selected(toks, ids)
            o = ora.forward(toks, head_mode=1, vocab_ids=ids)
            assert np.array_equal(g, o), (n, H.rel_l2(g, o))
        # decode width onto the 8300-token cache: 2 queries, then 1 (k_attn_dec_scores + k_attn_dec_pv)
        gpu.profile(True)
        gpu.profile_reset()
        try:
            for step in (rng.integers(0, cfg.vocab, 2), rng.integers(0, cfg.vocab, 1)):
                g = gpu.forward(step)
                o = ora.forward(step, head_mode=2)
                assert np.array_equal(g, o), H.rel_l2(g, o)
            assert gpu.profile_read("attn_decode")[0] == 2 * cfg.n_layer
        finally:
            gpu.profile(False)
    finally:
        gpu.close()


def test_non_finite_score_rows_take_the_uniform_softmax(shs, oracle):
    """Kernels.Softmax weighs every key of a row equally when the row's maximum is not
    finite (Kernels.cs:157-200). A huge attention-norm gain in layer 0 makes q·k overflow:
    at 1e19 some rows overflow and others stay finite, at 1e20 almost all overflow. The
    fused kernel (70 tokens; 1300, spilling score tiles past the LDS), the three-kernel path
    (8300 tokens, its items past 256 key tiles) and the decode-width kernels (one more token)
    must all match the oracle bit for bit."""
    cfg = oracle.make_config(**TINY)
    tensors, types = H.synth_model_tensors(oracle, cfg, 2, seed=7)
    rng = np.random.default_rng(23)
    ids = [3, 100, 400]
    flt_max = float(np.finfo(np.float32).max)
    for gain, mixed in ((1e19, True), (1e20, False)):
        t2 = dict(tensors)
        t2["blk.0.attn_norm.weight"] = (tensors["blk.0.attn_norm.weight"] * np.float32(gain)).astype(np.float32)
        gpu = shs.MinistralModel.from_tensors(H.shs_config_from_oracle(shs, cfg), t2, types)
        ora = oracle.OracleModel(cfg, t2, types, cap=8400)
        try:
            for n in (70, 1300, 8300):
                toks = rng.integers(0, cfg.vocab, n)
                gpu.reset_kv_cache()
                ora.reset()
                g = gpu.forward_selected(toks, ids)
                cap = {}
                o = ora.forward(toks, head_mode=1, vocab_ids=ids, capture=lambda nm, a: cap.__setitem__(nm, a))
                assert np.array_equal(g, o, equal_nan=True), (gain, n, H.rel_l2(g, o))
                # the premise: layer 0's unscaled scores (exact in float64) pass FLT_MAX in some rows
                # (checked over the first 1300 query rows)
                m_rows = min(n, 1300)
                q = cap["blk.0.q_rope"][:m_rows, :cfg.head_dim].astype(np.float64)
                k = cap["blk.0.k_rope"][:m_rows, :cfg.head_dim].astype(np.float64)
                s = np.abs(q @ k.T)
                row_max = np.array([s[i, :i + 1].max() for i in range(m_rows)])
                over = row_max > flt_max
                assert over.any(), (gain, n)
                if mixed:
                    assert not over.all(), (gain, n)
            step = rng.integers(0, cfg.vocab, 1)
            g = gpu.forward(step)
            o = ora.forward(step, head_mode=2)
            assert np.array_equal(g, o, equal_nan=True), (gain, H.rel_l2(g, o))
        finally:
            gpu.close()


def test_two_handles_on_two_host_threads_match_their_serial_results(shs, oracle):
    """Separate handles may run concurrently, each on its own stream (ShieldstralModerator.cs:46,
    MinistralModel.cs:21-22): two handles of a model, driven from two host threads at once
    through prefill and decode, give the same bits as each run alone. The first passes raise
    the kernels' LDS limits, which the two threads share."""
    import threading

    cfg = oracle.make_config(n_layer=2, hidden=256, n_head=4, n_kv_head=1, head_dim=128, ffn=512, vocab=512)
    tensors, types = H.synth_model_tensors(oracle, cfg, 2, seed=29)
    rng = np.random.default_rng(31)
    prompts = [rng.integers(0, cfg.vocab, n) for n in (600, 1200)]
    steps = [rng.integers(0, cfg.vocab, 3) for _ in prompts]
    handles = [shs.MinistralModel.from_tensors(H.shs_config_from_oracle(shs, cfg), tensors, types) for _ in prompts]

    def run(m, prompt, step):
        m.reset_kv_cache()
        out = [m.forward(prompt)]
        for t in step:
            out.append(m.forward([t]))
        return out

    try:
        serial = [run(m, p, st) for m, p, st in zip(handles, prompts, steps)]
        results = [None, None]
        errors = []
        barrier = threading.Barrier(2)

        def worker(i):
            try:
                barrier.wait()
                for _ in range(3):
                    results[i] = run(handles[i], prompts[i], steps[i])
            except Exception as e:  # reported below
                errors.append(e)

        threads = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
        for th in threads:
            th.start()
        for th in threads:
            th.join()
        assert not errors, errors
        for i in range(2):
            for a, b in zip(results[i], serial[i]):
                assert np.array_equal(a, b), i
    finally:
        for m in handles:
            m.close()


def test_packed_batch_of_decode_width_prompts_matches_the_oracle(shs, oracle, tiny):
    """A packed batch of 1-4-token prompts: every item is decode width, so attention runs
    k_attn_dec_scores + k_attn_dec_pv over 5 items, while the GEMMs (T = 12 > 4) take k_gemm:
    both widths meet in one pass."""
    cfg, tensors, types, gpu, ora = tiny
    rng = np.random.default_rng(19)
    prompts = [rng.integers(0, cfg.vocab, n) for n in (1, 4, 2, 3, 2)]
    ids = [5, 6, 500]
    batch = gpu.forward_batch(prompts, ids)
    for p, row in zip(prompts, batch):
        ora.reset()
        assert np.array_equal(row, ora.forward(p, head_mode=1, vocab_ids=ids))


def test_selected_rows_are_bit_identical_to_the_full_head(shs, tiny):
    """SystemPromptCacheTests.ScoringReadsExactlyWhatTheFullHeadWouldHave."""
    cfg, tensors, types, gpu, ora = tiny
    toks = np.random.default_rng(2).integers(0, cfg.vocab, 40)
    ids = [3, 400, 3, 511, 0]
    gpu.reset_kv_cache()
    full = gpu.forward(toks)
    gpu.reset_kv_cache()
    sel = gpu.forward_selected(toks, ids)
    assert np.array_equal(sel, full[ids])
    # 70000 ids (280 KB) do not fit the library's pinned upload staging: that upload takes the
    # direct, waited copy, and the rows are still the full head's
    many = np.random.default_rng(3).integers(0, cfg.vocab, 70000)
    gpu.reset_kv_cache()
    sel = gpu.forward_selected(toks, many)
    assert np.array_equal(sel, full[many])


def test_single_token_decode_matches_the_oracle(shs, tiny):
    """Benchmark.cs:399-410's decode: single-token forwards (full-vocabulary logits) onto a
    prefilled cache, then a 3-token step — the narrow GEMM path with unfused RoPE and SwiGLU
    — bit-exact against the oracle stepping its own cache the same way."""
    cfg, tensors, types, gpu, ora = tiny
    toks = np.random.default_rng(12).integers(0, cfg.vocab, 60)
    gpu.reset_kv_cache()
    ora.reset()
    assert np.array_equal(gpu.forward(toks[:50]), ora.forward(toks[:50], head_mode=2))
    for i in range(50, 57):
        g = gpu.forward(toks[i:i + 1])
        o = ora.forward(toks[i:i + 1], head_mode=2)
        assert np.array_equal(g.view(np.uint32), o.view(np.uint32)), i
    last = gpu.forward(toks[57:60])
    assert np.array_equal(last, ora.forward(toks[57:60], head_mode=2))
    assert gpu.cached_token_count == 60
    gpu.reset_kv_cache()
    assert np.array_equal(gpu.forward(toks), last)  # the same position through the wide kernels


@pytest.mark.parametrize("qt", [3, 6, 7, 8])
def test_decode_with_other_weight_types(shs, oracle, qt):
    """The narrow kernels' fused q|k|v (RoPE, KV store) and gate|up (SwiGLU, quantization)
    epilogues for the offset (Q4_1, Q5_1), fifth-bit (Q5_0, Q5_1) and Q8_0 types: a prompt,
    then 1-, 2- and 4-token steps, bit-exact against the oracle."""
    cfg = oracle.make_config(**TINY)
    tensors, types = H.synth_model_tensors(oracle, cfg, qt, seed=40 + qt)
    gpu = shs.MinistralModel.from_tensors(H.shs_config_from_oracle(shs, cfg), tensors, types)
    ora = oracle.OracleModel(cfg, tensors, types, cap=200)
    try:
        toks = np.random.default_rng(qt).integers(0, cfg.vocab, 47)
        assert np.array_equal(gpu.forward(toks[:40]), ora.forward(toks[:40], head_mode=2))
        for a, b in ((40, 41), (41, 43), (43, 47)):
            g = gpu.forward(toks[a:b])
            o = ora.forward(toks[a:b], head_mode=2)
            assert np.array_equal(g.view(np.uint32), o.view(np.uint32)), (qt, a, b, H.rel_l2(g, o))
    finally:
        gpu.close()


def test_prefix_cache_is_bit_identical(shs, tiny):
    """SystemPromptCacheTests.CachedAndUncachedProduceIdenticalLogits (all vocab entries)."""
    cfg, tensors, types, gpu, ora = tiny
    toks = np.random.default_rng(3).integers(0, cfg.vocab, 90)
    gpu.reset_kv_cache()
    full = gpu.forward(toks)
    cache = shs.SystemPromptCache.capture(gpu, toks[:37])
    assert gpu.cached_token_count == 37
    cache.restore_into(gpu)
    cached = gpu.forward(toks[37:])
    assert np.array_equal(full, cached)
    assert gpu.cached_token_count == 90


def test_kv_snapshot_layout_matches_the_oracle(shs, tiny):
    cfg, tensors, types, gpu, ora = tiny
    toks = np.random.default_rng(4).integers(0, cfg.vocab, 45)
    gpu.reset_kv_cache()
    gpu.prefill(toks)
    ora.reset()
    ora.forward(toks, head_mode=0)
    snap = gpu.kv_cache.snapshot(45)
    ref = ora.snapshot(45)
    assert snap.shape == ref.shape
    assert np.array_equal(snap, ref)
    with pytest.raises(shs.ArgumentOutOfRangeError):
        gpu.kv_cache.snapshot(46)
    with pytest.raises(shs.ArgumentError):
        gpu.kv_cache.restore(snap[:-1], 45)


def test_kv_cache_grows_without_changing_results(shs, oracle, tiny):
    cfg, tensors, types, gpu, ora = tiny
    small = shs.MinistralModel.from_tensors(H.shs_config_from_oracle(shs, cfg), tensors, types, initial_cache_capacity=8)
    toks = np.random.default_rng(5).integers(0, cfg.vocab, 70)
    small.prefill(toks[:30])
    grown = small.forward(toks[30:])
    assert small.kv_cache.capacity >= 70
    gpu.reset_kv_cache()
    assert np.array_equal(grown, gpu.forward(toks))
    small.close()


def test_a_cancelled_pass_leaves_the_instance_usable(shs, tiny):
    """ModerationCancellationTests: cancellation is observed, the KV length does not move,
    and the next request scores exactly as a fresh one."""
    cfg, tensors, types, gpu, ora = tiny
    toks = np.random.default_rng(6).integers(0, cfg.vocab, 50)
    gpu.reset_kv_cache()
    gpu.prefill(toks[:10])
    flag = shs.CancellationFlag()
    flag.cancel()
    with pytest.raises(shs.OperationCanceledError):
        gpu.forward_selected(toks[10:], [1, 2], cancel=flag)
    assert gpu.cached_token_count == 10
    after = gpu.forward_selected(toks[10:], [1, 2])
    gpu.reset_kv_cache()
    assert np.array_equal(after, gpu.forward_selected(toks, [1, 2]))


def test_invalid_requests_raise_the_reference_exceptions(shs, tiny):
    cfg, tensors, types, gpu, ora = tiny
    gpu.reset_kv_cache()
    with pytest.raises(shs.ArgumentOutOfRangeError):
        gpu.forward_selected([1, 2, cfg.vocab], [0])
    with pytest.raises(shs.ArgumentOutOfRangeError):
        gpu.forward_selected([1, 2], [cfg.vocab])
    with pytest.raises(shs.ArgumentError):
        gpu.forward_selected([], [0])
    assert gpu.cached_token_count == 0


def test_packed_ragged_batch_equals_one_prompt_at_a_time(shs, oracle, tiny):
    cfg, tensors, types, gpu, ora = tiny
    rng = np.random.default_rng(7)
    prompts = [rng.integers(0, cfg.vocab, n) for n in (5, 64, 33, 100, 1)]
    ids = [7, 8, 9]
    batch = gpu.forward_batch(prompts, ids)
    for p, row in zip(prompts, batch):
        gpu.reset_kv_cache()
        assert np.array_equal(gpu.forward_selected(p, ids), row)
        ora.reset()
        assert np.array_equal(row, ora.forward(p, head_mode=1, vocab_ids=ids))


def test_moderator_scores_like_the_oracle(shs, oracle, tiny):
    cfg, tensors, types, gpu, ora = tiny
    rng = np.random.default_rng(8)
    prefix = rng.integers(0, cfg.vocab, 12)
    yes, no = [10, 11, 12], [20, 21]
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "prefix.shkv")
        mod = shs.ShieldstralModerator(gpu, yes, no, system_prefix_tokens=prefix, prefix_cache_path=path)
        assert os.path.exists(path) and mod.cached_prefix_tokens == 12
        again = shs.SystemPromptCache.try_load(path, gpu)
        assert again is not None and np.array_equal(again.state, mod._prefix.state)
        prompt = np.concatenate([prefix, rng.integers(0, cfg.vocab, 40)])
        r = mod.moderate_tokens(prompt)
        assert r.prefilled_tokens == 12 and r.prompt_tokens == 52
        ora.reset()
        logits = ora.forward(prompt, head_mode=1, vocab_ids=yes + no)
        s, y, n = oracle.score(logits, 3, 2)
        assert r.yes_logit == y and r.no_logit == n
        assert abs(r.score - s) < 1e-6
        assert r.is_unsafe == (r.score > 0.5) and r.is_unsafe_at(0.0) == (r.score > 0.0)
        other = rng.integers(0, cfg.vocab, 30)  # no shared prefix: the cache is reset, not restored
        r2 = mod.moderate_tokens(other)
        assert r2.prefilled_tokens == 0
        assert mod.top_verdict_token(prompt) == int(np.argmax(gpu.forward(prompt[12:])))


def test_gguf_file_loads_identically_and_bad_files_are_rejected(shs, oracle, tiny):
    import gguf_writer
    cfg, tensors, types, gpu, ora = tiny
    toks = np.random.default_rng(9).integers(0, cfg.vocab, 30)
    gpu.reset_kv_cache()
    ref = gpu.forward(toks)
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "tiny.gguf")
        gguf_writer.write_gguf(path, "mistral3", cfg, tensors, types)
        m = shs.MinistralModel.open(path)
        assert m.config.vocab_size == cfg.vocab and m.config.layer_count == cfg.n_layer
        assert np.array_equal(m.forward(toks), ref)
        m.close()
        bad = os.path.join(d, "trunc.gguf")
        gguf_writer.write_gguf(bad, "mistral3", cfg, tensors, types, truncate_by=100)
        with pytest.raises(shs.ModelIOError):
            shs.MinistralModel.open(bad)
        junk = os.path.join(d, "junk.gguf")
        with open(junk, "wb") as f:
            f.write(b"not a gguf at all, just some bytes")
        with pytest.raises(shs.InvalidDataError):
            shs.MinistralModel.open(junk)
        other = os.path.join(d, "other.gguf")
        gguf_writer.write_gguf(other, "gemma3", cfg, tensors, types)
        with pytest.raises(shs.NotSupportedError):
            shs.MinistralModel.open(other)
        missing = dict(tensors)
        del missing["blk.1.ffn_up.weight"]
        gone = os.path.join(d, "missing.gguf")
        gguf_writer.write_gguf(gone, "mistral3", cfg, missing, types)
        with pytest.raises(shs.TensorNotFoundError):
            shs.MinistralModel.open(gone)


def test_one_full_size_decoder_layer_t512(shs, oracle):
    """One decoder layer at T=512 on X ~ N(0,1): RMSNorm (gain N(1,0.1)), Q4_0 q/k/v, RoPE θ=1e6,
    GQA 32/8, o-proj + residual, RMSNorm, SwiGLU FFN 9216 + residual."""
    cfg = oracle.make_config(n_layer=1, vocab=64)
    tensors, types = H.synth_model_tensors(oracle, cfg, 2, seed=33)
    gpu = shs.MinistralModel.from_tensors(H.shs_config_from_oracle(shs, cfg), tensors, types)
    x = np.random.default_rng(34).standard_normal((512, 3072)).astype(np.float32)
    y = gpu.layer_forward(0, x)
    ora = oracle.OracleModel(cfg, tensors, types, cap=512)
    ref = ora.layer_forward(0, x)
    assert np.array_equal(y, ref), H.rel_l2(y, ref)
    gpu.close()


def test_synthetic_model_round_trips_through_download(shs, oracle):
    cfg = oracle.make_config(n_layer=2, hidden=256, n_head=8, n_kv_head=2, ffn=768, vocab=1000)
    scfg = H.shs_config_from_oracle(shs, cfg)
    syn = shs.MinistralModel.synthetic(scfg, shs.Q5_1, shs.Q4_0, seed=5)
    names = list(scfg.tensor_shapes(shs.Q5_1, shs.Q4_0))
    tensors = {n: syn.download(n) for n in names}
    types = {n: (0 if n.endswith("norm.weight") else (2 if n == "token_embd.weight" else 7)) for n in names}
    w = oracle.dequantize(7, tensors["blk.0.ffn_gate.weight"], 768 * 256)
    assert abs(float(np.std(w)) - 0.02) < 0.002 and abs(float(np.mean(w))) < 0.002
    g = tensors["blk.1.attn_norm.weight"]
    assert abs(float(np.mean(g)) - 1.0) < 0.03 and abs(float(np.std(g)) - 0.1) < 0.03
    again = shs.MinistralModel.from_tensors(scfg, tensors, types)
    toks = np.random.default_rng(10).integers(0, cfg.vocab, 64)
    a = syn.forward(toks)
    b = again.forward(toks)
    assert np.array_equal(a, b)
    ora = oracle.OracleModel(cfg, tensors, types, cap=64)
    assert np.array_equal(a, ora.forward(toks, head_mode=2))
    syn.close()
    again.close()


def test_wide_hidden_rows_take_the_one_row_rmsnorm_blocks(shs, oracle):
    """A hidden size of 5120: four rows' LDS (the row and its transposed squares) no longer fit
    160 KB, so the RMSNorm launches run one row per block; the model stays bit-exact."""
    cfg = oracle.make_config(n_layer=1, hidden=5120, n_head=40, n_kv_head=10, head_dim=128, ffn=1024, vocab=512)
    scfg = H.shs_config_from_oracle(shs, cfg)
    syn = shs.MinistralModel.synthetic(scfg, shs.Q4_0, shs.Q4_0, seed=8)
    names = list(scfg.tensor_shapes(shs.Q4_0, shs.Q4_0))
    tensors = {n: syn.download(n) for n in names}
    types = {n: (0 if n.endswith("norm.weight") else 2) for n in names}
    toks = np.random.default_rng(13).integers(0, cfg.vocab, 45)
    got = syn.forward(toks)
    ora = oracle.OracleModel(cfg, tensors, types, cap=64)
    assert np.array_equal(got, ora.forward(toks, head_mode=2))
    syn.close()


def test_device_exp_is_the_oracle_exp_bit_for_bit(shs, oracle):
    rng = np.random.default_rng(12)
    x = np.concatenate([np.linspace(-110, 90, 400001, dtype=np.float32),
                        (rng.standard_normal(200000) * 30).astype(np.float32),
                        np.array([0.0, -0.0, -104.0, -103.99, -87.5, 88.72, 88.73, np.inf, -np.inf], np.float32)])
    got = shs.device_expf(x)
    lib = oracle.lib()
    ref = np.array([lib.ora_expf(float(v)) for v in x], np.float32)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


YARN = dict(rope_scale=16.0, rope_orig_ctx=16, yarn_active=1, yarn_beta_fast=32.0, yarn_beta_slow=1.0,
            yarn_ext_factor=1.0, yarn_mscale=1.0, yarn_mscale_all_dim=1.0, attn_temperature=0.1)


def test_the_real_checkpoints_rope_keys_run_yarn_and_the_query_temperature(shs, oracle, tmp_path):
    """A GGUF carrying the converter's YaRN and temperature keys
    (tools/convert_shieldstral_to_gguf.py:307-323), opened through shs_open: YarnActive
    (ModelConfig.cs:54-56), the YaRN frequencies (Rope.cs:33-106) and, with a 16-token
    original context, the Llama-4 query temperature from position 16 on
    (MinistralModel.cs:471-482). A 40-token prefill (every capture), then 1-, 2- and
    4-token steps and the KV cache, bit-exact against the oracle."""
    import gguf_writer as GW
    cfg = oracle.make_config(n_layer=2, hidden=256, n_head=8, n_kv_head=2, head_dim=128, ffn=512, vocab=512, **YARN)
    tensors, types = H.synth_model_tensors(oracle, cfg, 2, seed=61)
    path = tmp_path / "yarn.gguf"
    GW.write_gguf(path, "mistral3", cfg, tensors, types, extra_kv=GW.yarn_keys("mistral3", cfg))
    gpu = shs.MinistralModel.open(str(path), initial_cache_capacity=64)
    ora = oracle.OracleModel(cfg, tensors, types, cap=64)
    try:
        c = gpu.config
        assert c.yarn_active and c.rope_original_context_length == 16 and c.attention_temperature_scale > 0
        toks = np.random.default_rng(8).integers(0, cfg.vocab, 47)
        gcap, ocap = {}, {}
        gpu.set_capture(lambda n, a: gcap.__setitem__(n, a))
        try:
            g = gpu.forward(toks[:40])
        finally:
            gpu.set_capture(None)
        o = ora.forward(toks[:40], head_mode=2, capture=lambda n, a: ocap.__setitem__(n, a))
        assert set(gcap) == set(ocap)
        for name in sorted(gcap):
            assert np.array_equal(gcap[name], ocap[name]), name
        assert np.array_equal(g, o)
        for a, b in ((40, 41), (41, 43), (43, 47)):
            g = gpu.forward(toks[a:b])
            o = ora.forward(toks[a:b], head_mode=2)
            assert np.array_equal(g.view(np.uint32), o.view(np.uint32)), (a, b)
        assert np.array_equal(gpu.kv_cache.snapshot(47), ora.snapshot(47))
    finally:
        gpu.close()


def test_decode_at_the_full_layer_width_matches_the_oracle(shs, oracle):
    """The decode-width kernels at the real layer shape (hidden 3072, FFN 9216, 32 query and
    8 KV heads; two layers, 4096-entry vocabulary): the q|k|v and gate|up kernels that
    normalize their own input row (96 blocks: the 16-step register rounds iterate), the
    fused RoPE/KV-store and SwiGLU epilogues and the decode attention with 8 KV heads. A
    40-token prefill, then 1-, 2- and 4-token steps: full logits and the KV cache bit-exact."""
    cfg = oracle.make_config(n_layer=2, hidden=3072, n_head=32, n_kv_head=8, head_dim=128, ffn=9216, vocab=4096)
    tensors, types = H.synth_model_tensors(oracle, cfg, 2, seed=62)
    gpu = shs.MinistralModel.from_tensors(H.shs_config_from_oracle(shs, cfg), tensors, types,
                                          initial_cache_capacity=64)
    ora = oracle.OracleModel(cfg, tensors, types, cap=64)
    try:
        toks = np.random.default_rng(9).integers(0, cfg.vocab, 47)
        assert np.array_equal(gpu.forward(toks[:40]), ora.forward(toks[:40], head_mode=2))
        for a, b in ((40, 41), (41, 42), (42, 44), (44, 47)):
            g = gpu.forward(toks[a:b])
            o = ora.forward(toks[a:b], head_mode=2)
            assert np.array_equal(g.view(np.uint32), o.view(np.uint32)), (a, b, H.rel_l2(g, o))
            assert np.array_equal(gpu.kv_cache.snapshot(b), ora.snapshot(b)), (a, b)
    finally:
        gpu.close()


def test_a_cancel_set_while_the_layers_run_is_observed(shs, tiny):
    """ModerationCancellationTests.cs:50-74: the flag is set after layer 0 has run on the
    GPU (from the activation callback, so the moment is exact), and the pass stops before
    layer 1 with OperationCanceledError; the KV length does not move and the next request
    scores exactly like a fresh one."""
    cfg, tensors, types, gpu, ora = tiny
    toks = np.random.default_rng(13).integers(0, cfg.vocab, 60)
    gpu.reset_kv_cache()
    expected = gpu.forward_selected(toks, [4, 9])
    gpu.reset_kv_cache()
    gpu.prefill(toks[:12])
    flag = shs.CancellationFlag()
    seen = []

    def sink(name, arr):
        seen.append(name)
        if name == "blk.0.output":
            flag.cancel()

    gpu.set_capture(sink)
    try:
        with pytest.raises(shs.OperationCanceledError):
            gpu.forward_selected(toks[12:], [4, 9], cancel=flag)
    finally:
        gpu.set_capture(None)
    assert "blk.0.output" in seen and not any(n.startswith("blk.1.") for n in seen)
    assert gpu.cached_token_count == 12
    assert np.array_equal(gpu.forward_selected(toks[12:], [4, 9]), expected)

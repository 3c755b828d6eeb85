"""Full Shieldstral-3B-shaped random-init model (26 layers, 3072/9216, 32/8 heads, vocab
131072): the 1024-token Q4_0 verdict and the 16-prompt ragged Q5_1 batch.

Both are checked against the oracle at full size: the verdict's logits and its whole KV
cache bit for bit, and, from the ragged batch, its longest prompt (1800 tokens: past the 35
key tiles a block's LDS holds, so the fused attention spills its later score tiles to the
item's scratch region) and its shortest (90).
The oracle runs on the host's threads on the weight bytes downloaded from the device;
each of these takes well under a minute there. Size-independent properties back them:
determinism, selected rows = full head, prefix cache = full pass, batch = single."""
import os

import numpy as np
import pytest

import helpers as H

pytestmark = pytest.mark.gpu


def oracle_of(shs, oracle, model, weight_type, cap):
    """The oracle model over the exact bytes the device holds."""
    cfg = model.config
    ocfg = oracle.make_config(n_layer=cfg.layer_count, hidden=cfg.hidden_size, n_head=cfg.head_count,
                              n_kv_head=cfg.kv_head_count, head_dim=cfg.head_dim, ffn=cfg.feed_forward_size,
                              vocab=cfg.vocab_size, eps=cfg.rms_norm_eps, rope_theta=cfg.rope_freq_base,
                              rope_dim=cfg.rope_dim)
    names = list(cfg.tensor_shapes(weight_type, weight_type))
    tensors = {n: model.download(n) for n in names}
    types = {n: (0 if n.endswith("norm.weight") else weight_type) for n in names}
    return oracle.OracleModel(ocfg, tensors, types, cap=cap)


@pytest.fixture(scope="module")
def full_q4(shs):
    m = shs.MinistralModel.synthetic(shs.SHIELDSTRAL_3B, shs.Q4_0, seed=2024, initial_cache_capacity=1024)
    yield m
    m.close()


def test_1024_token_verdict_properties(shs, full_q4):
    m = full_q4
    rng = np.random.default_rng(1024)
    toks = rng.integers(0, 131072, 1024)
    yes, no = rng.choice(131072, 2, replace=False)
    ids = [int(yes), int(no)]
    m.reset_kv_cache()
    sel = m.forward_selected(toks, ids)
    m.reset_kv_cache()
    sel2 = m.forward_selected(toks, ids)
    assert np.array_equal(sel, sel2) and np.all(np.isfinite(sel))
    m.reset_kv_cache()
    full = m.forward(toks)
    assert np.array_equal(full[ids], sel)
    m.reset_kv_cache()
    m.prefill(toks[:300])
    assert np.array_equal(m.forward_selected(toks[300:], ids), sel)
    r = shs.score(sel, 1, 1024, 0)
    assert 0.0 <= r.score <= 1.0
    assert abs(r.score - 1 / (1 + np.exp(-(float(sel[0]) - float(sel[1]))))) < 1e-6
    assert np.array_equal(m.forward_batch([toks], ids)[0], sel)


def test_ragged_q5_1_batch_of_16_prompts(shs):
    m = shs.MinistralModel.synthetic(shs.SHIELDSTRAL_3B, shs.Q5_1, seed=5, initial_cache_capacity=2048)
    rng = np.random.default_rng(16)
    lens = rng.integers(64, 2049, 16)
    prompts = [rng.integers(0, 131072, n) for n in lens]
    ids = [int(i) for i in rng.choice(131072, 2, replace=False)]
    batch = m.forward_batch(prompts, ids)
    for p, row in zip(prompts, batch):
        m.reset_kv_cache()
        assert np.array_equal(m.forward_selected(p, ids), row)
    scores = [shs.score(row, 1, len(p), 0).score for p, row in zip(prompts, batch)]
    assert all(0.0 <= s <= 1.0 for s in scores)
    m.close()


@pytest.mark.timeout(600)
def test_1024_token_verdict_matches_the_oracle(shs, oracle, full_q4):
    """The Q4_0 verdict workload, 26 layers at T = 1024: yes/no logits and the 26-layer KV
    cache (218 MB) bit-identical to the oracle's."""
    m = full_q4
    rng = np.random.default_rng(1024)
    toks = rng.integers(0, 131072, 1024)
    ids = [int(i) for i in rng.choice(131072, 2, replace=False)]
    m.reset_kv_cache()
    sel = m.forward_selected(toks, ids)
    snap = m.kv_cache.snapshot(1024)
    ora = oracle_of(shs, oracle, m, shs.Q4_0, 1024)
    ref = ora.forward(toks, head_mode=1, vocab_ids=ids, threads=min(16, os.cpu_count() or 1))
    assert np.array_equal(sel.view(np.uint32), ref.view(np.uint32))
    assert np.array_equal(snap.view(np.uint32), ora.snapshot(1024).view(np.uint32))


@pytest.mark.timeout(900)
def test_ragged_q5_1_batch_longest_and_shortest_prompts_match_the_oracle(shs, oracle):
    m = shs.MinistralModel.synthetic(shs.SHIELDSTRAL_3B, shs.Q5_1, seed=5, initial_cache_capacity=2048)
    try:
        rng = np.random.default_rng(16)
        lens = rng.integers(64, 2049, 16)
        prompts = [rng.integers(0, 131072, n) for n in lens]
        ids = [int(i) for i in rng.choice(131072, 2, replace=False)]
        batch = m.forward_batch(prompts, ids)
        ora = oracle_of(shs, oracle, m, shs.Q5_1, int(lens.max()))
        for s in (int(np.argmax(lens)), int(np.argmin(lens))):
            ora.reset()
            ref = ora.forward(prompts[s], head_mode=1, vocab_ids=ids, threads=min(16, os.cpu_count() or 1))
            assert np.array_equal(batch[s].view(np.uint32), ref.view(np.uint32)), (s, int(lens[s]))
    finally:
        m.close()


def test_a_cancel_from_another_thread_stops_a_running_verdict(shs, full_q4):
    """ModerationCancellationTests.cs:50-74 on the full model: a thread sets the flag a few
    milliseconds into a 1024-token pass (about 14 ms of GPU work). The pass raises
    OperationCanceledError, the KV length stays at the prefilled 100 tokens, and the
    next verdict is bit-identical to an uncancelled one. Thread timing is not exact, so
    several delays are tried and at least one must land mid-pass."""
    import threading
    import time
    m = full_q4
    rng = np.random.default_rng(77)
    toks = rng.integers(0, 131072, 1124)
    ids = [11, 12]
    m.reset_kv_cache()
    m.prefill(toks[:100])
    expected = m.forward_selected(toks[100:], ids)
    cancelled = 0
    for delay_ms in (2.0, 4.0, 6.0):
        m.reset_kv_cache()
        m.prefill(toks[:100])
        flag = shs.CancellationFlag()
        t = threading.Thread(target=lambda: (time.sleep(delay_ms / 1e3), flag.cancel()))
        t.start()
        try:
            got = m.forward_selected(toks[100:], ids, cancel=flag)
            assert np.array_equal(got, expected)  # finished before the flag was set
            assert m.cached_token_count == 1124
        except shs.OperationCanceledError:
            cancelled += 1
            assert m.cached_token_count == 100
            assert np.array_equal(m.forward_selected(toks[100:], ids), expected)
        t.join()
    assert cancelled >= 1

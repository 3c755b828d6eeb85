"""Full Shieldstral-3B-shaped random-init model (26 layers, 3072/9216, 32/8 heads, vocab
131072): the 1024-token Q4_0 verdict and the 16-prompt ragged Q5_1 batch. At these sizes
the oracle would take minutes, so parity rests on size-independent properties: determinism,
selected-rows = full-head bit identity, prefix-cache bit identity, and batch = single."""
import numpy as np
import pytest

import helpers as H

pytestmark = pytest.mark.gpu


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

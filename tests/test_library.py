"""CPU-side checks of libshieldstral_hip: the C ABI is complete, errors map onto the
reference's exception types, and the host logic (Score, SHKV files, moderator plumbing)
behaves like llm-shield's. No GPU compute is launched here."""
import re
import struct
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "shieldstral_hip.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(shs_\w+)\s*\(", text)) - {"shs_capture_fn"})


def test_library_exports_every_declared_symbol(shs):
    lib = shs.load_library()
    declared = declared_functions()
    assert declared, "no declarations parsed"
    for name in declared:
        assert hasattr(lib, name), name
    assert sorted(shs.EXPORTS) == declared


def test_product_library_does_not_link_the_oracle():
    import subprocess
    out = subprocess.run(["ldd", str(ROOT / "llm-shield_amd" / "libshieldstral_hip.so")], capture_output=True,
                         text=True).stdout
    assert "oracle" not in out
    syms = subprocess.run(["nm", "-D", str(ROOT / "llm-shield_amd" / "libshieldstral_hip.so")], capture_output=True,
                          text=True).stdout
    assert "ora_" not in syms


def test_unsupported_weight_type_is_rejected_before_touching_a_device(shs):
    with pytest.raises(shs.NotSupportedError, match="Q4_K|unsupported|no integer GEMM"):
        shs.WeightMatrix(12, 32, 256, np.zeros(32 * 8 * 144, np.uint8))


def test_bad_shapes_are_argument_errors(shs):
    with pytest.raises(shs.ArgumentError):
        shs.WeightMatrix(2, 32, 100, np.zeros(32 * 4 * 18, np.uint8))


def test_missing_file_is_an_io_error(shs, tmp_path):
    with pytest.raises(shs.ModelIOError):
        shs.MinistralModel.open(str(tmp_path / "nope.gguf"))


def test_score_matches_the_reference_closed_form(shs):
    """ShieldstralModerator.Score: best yes vs best no, two-way softmax."""
    r = shs.score(np.array([1.5, 4.0, 2.0, -1.0, 3.0], np.float32), 3, 100, 20)
    assert r.yes_logit == 4.0 and r.no_logit == 3.0
    assert abs(r.score - 1 / (1 + np.exp(-1.0))) < 1e-7
    assert r.is_unsafe and r.is_unsafe_at(0.7) and not r.is_unsafe_at(0.8)
    assert r.prompt_tokens == 100 and r.prefilled_tokens == 20
    big = shs.score(np.array([1000.0, -1000.0], np.float32), 1, 1, 0)
    assert big.score == 1.0 and np.isfinite(big.score)
    assert str(r).startswith("UNSAFE score=")


class _FakeModel:
    """Enough of MinistralModel for SystemPromptCache's file handling."""

    def __init__(self, shs, path=""):
        self.model_path = path
        self.config = shs.SHIELDSTRAL_3B


def test_shkv_round_trip_and_rejections(shs, tmp_path):
    m = _FakeModel(shs)
    tokens = np.array([1, 2, 3, 4], np.int32)
    state = np.random.default_rng(0).standard_normal(2 * 26 * 8 * 4 * 128).astype(np.float32)
    fp = shs.SystemPromptCache.compute_fingerprint(m, tokens)
    c = shs.SystemPromptCache(tokens, state, fp)
    path = tmp_path / "p.shkv"
    c.save(path)
    raw = path.read_bytes()
    assert struct.unpack("<Ii", raw[:8]) == (0x53484B56, 1)
    assert raw[8] == 64  # 7-bit length prefix of a 64-hex-digit fingerprint
    back = shs.SystemPromptCache.try_load(path, m)
    assert back is not None and np.array_equal(back.tokens, tokens) and np.array_equal(back.state, state)
    assert back.is_prefix_of([1, 2, 3, 4, 9]) and not back.is_prefix_of([1, 2, 3]) and not back.is_prefix_of([1, 2, 4, 4])
    other = _FakeModel(shs, "elsewhere.gguf")
    assert shs.SystemPromptCache.try_load(path, other) is None
    path.write_bytes(raw[:-10])
    assert shs.SystemPromptCache.try_load(path, m) is None
    path.write_bytes(b"XXXX" + raw[4:])
    assert shs.SystemPromptCache.try_load(path, m) is None
    assert shs.SystemPromptCache.try_load(tmp_path / "absent.shkv", m) is None


def test_moderator_requires_yes_and_no_tokens(shs):
    with pytest.raises(shs.InvalidDataError):
        shs.ShieldstralModerator(_FakeModel(shs), [], [1])


def test_config_tensor_table_matches_the_reference_names(shs):
    t = shs.SHIELDSTRAL_3B.tensor_shapes(shs.Q4_0, shs.Q4_0)
    assert len(t) == 2 + 9 * 26  # GgufReaderTests: 236 tensors
    assert t["blk.0.attn_q.weight"][1:] == (3072, 4096)
    assert t["blk.25.ffn_down.weight"][1:] == (9216, 3072)
    assert t["token_embd.weight"][1:] == (3072, 131072)

"""CPU-side checks of libshieldstral_hip: the C ABI is complete, errors map onto the
reference's exception types, and the host logic (Score, SHKV files, moderator plumbing)
behaves like llm-shield's. No GPU compute is launched here."""
import re
import struct
from pathlib import Path

import numpy as np
import pytest

import helpers as H

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


# ------------------------------------------------------------ GGUF header (CPU)

def _tiny_gguf(oracle, tmp_path, name="m.gguf", arch="mistral3", cfg_kw=None, **kw):
    import gguf_writer as GW
    cfg = oracle.make_config(n_layer=1, hidden=64, n_head=2, n_kv_head=1, head_dim=32, ffn=96, vocab=64,
                             rope_dim=32, **(cfg_kw or {}))
    tensors, types = H.synth_model_tensors(oracle, cfg, 2, seed=1)
    path = tmp_path / name
    GW.write_gguf(path, arch, cfg, tensors, types, **kw)
    return path, cfg


def test_read_config_follows_model_config_from_gguf(shs, oracle, tmp_path):
    """ModelConfig.FromGguf on the header alone: hyperparameters, the architecture
    string, and the converter's YaRN + temperature keys (YarnActive)."""
    import gguf_writer as GW
    yarn = dict(rope_scale=16.0, rope_orig_ctx=16, yarn_active=1, yarn_beta_fast=32.0, yarn_beta_slow=1.0,
                yarn_mscale=1.0, yarn_mscale_all_dim=1.0, attn_temperature=0.1)
    plain, _ = _tiny_gguf(oracle, tmp_path)
    c = shs.ModelConfig.from_gguf(plain)
    assert (c.layer_count, c.hidden_size, c.head_count, c.kv_head_count, c.head_dim) == (1, 64, 2, 1, 32)
    assert c.vocab_size == 64 and c.architecture == "mistral3" and not c.yarn_active
    cfg = oracle.make_config(n_layer=1, hidden=64, n_head=2, n_kv_head=1, head_dim=32, ffn=96, vocab=64,
                             rope_dim=32, **yarn)
    path, _ = _tiny_gguf(oracle, tmp_path, "y.gguf", arch="ministral3", cfg_kw=yarn,
                         extra_kv=GW.yarn_keys("ministral3", cfg))
    y = shs.ModelConfig.from_gguf(path)
    assert y.architecture == "ministral3" and y.yarn_active
    assert (y.rope_scale_factor, y.rope_original_context_length) == (16.0, 16)
    assert (y.yarn_mscale, y.yarn_mscale_all_dim) == (1.0, 1.0)
    assert y.attention_temperature_scale == pytest.approx(0.1)
    assert (y.yarn_beta_fast, y.yarn_beta_slow, y.yarn_ext_factor, y.rope_attn_factor) == (32.0, 1.0, 1.0, 1.0)


def test_damaged_headers_are_rejected_without_crashing(shs, oracle, tmp_path):
    """A string length near 2^64, a tensor offset that would wrap past the end of the
    address space, a fractional or zero general.alignment, and a header cut short: each
    is an InvalidDataError or ModelIOError, never a crash (GgufFile.cs:110-172)."""
    import struct as S
    import gguf_writer as GW
    good, _ = _tiny_gguf(oracle, tmp_path)
    raw = bytearray(good.read_bytes())
    # the first metadata key's length field sits right after the 24-byte header
    bad = bytearray(raw)
    bad[24:32] = S.pack("<Q", 2 ** 64 - 3)
    p = tmp_path / "strlen.gguf"
    p.write_bytes(bad)
    with pytest.raises((shs.InvalidDataError, shs.ModelIOError)):
        shs.ModelConfig.from_gguf(p)
    for off in (2 ** 64 - 8, 2 ** 63, len(raw)):
        p, _ = _tiny_gguf(oracle, tmp_path, f"off{off}.gguf", offset_override={"blk.0.ffn_down.weight": off})
        with pytest.raises(shs.ModelIOError):
            shs.ModelConfig.from_gguf(p)
    for akv in ((GW.F32, 0.5), (GW.U32, 0), (GW.F32, 1.5), (GW.STR, "32")):
        p, _ = _tiny_gguf(oracle, tmp_path, "align.gguf", alignment_kv=akv)
        with pytest.raises(shs.InvalidDataError):
            shs.ModelConfig.from_gguf(p)
    for cut in (30, len(raw) // 3):
        p = tmp_path / "cut.gguf"
        p.write_bytes(raw[:cut])
        with pytest.raises((shs.InvalidDataError, shs.ModelIOError)):
            shs.ModelConfig.from_gguf(p)
    p, _ = _tiny_gguf(oracle, tmp_path, "short.gguf", truncate_by=40)
    with pytest.raises(shs.ModelIOError, match="truncated"):
        shs.ModelConfig.from_gguf(p)
    assert shs.ModelConfig.from_gguf(good).hidden_size == 64


def test_shkv_fingerprint_carries_the_architecture(shs, oracle, tmp_path):
    """ComputeFingerprint appends Config.Architecture (SystemPromptCache.cs:90-105): a
    ministral3 GGUF's snapshot reloads against that model and its fingerprint is the
    SHA-256 of the reference's string with "ministral3" in it."""
    import hashlib
    import os
    path, _ = _tiny_gguf(oracle, tmp_path, "mini.gguf", arch="ministral3")
    m = _FakeModel(shs, str(path))
    m.config = shs.ModelConfig.from_gguf(path)
    toks = np.array([5, 6, 7], np.int32)
    fp = shs.SystemPromptCache.compute_fingerprint(m, toks)
    st = os.stat(path)
    ticks = st.st_mtime_ns // 100 + 621355968000000000
    ref = f"mini.gguf|{st.st_size}|{ticks}|ministral3|1x1x32|3:5,6,7,"
    assert fp == hashlib.sha256(ref.encode()).hexdigest()
    state = np.arange(2 * 1 * 1 * 3 * 32, dtype=np.float32)
    cache = shs.SystemPromptCache(toks, state, fp)
    cache.save(tmp_path / "mini.shkv")
    back = shs.SystemPromptCache.try_load(tmp_path / "mini.shkv", m)
    assert back is not None and back.fingerprint == fp and np.array_equal(back.state, state)
    m.config.architecture = "mistral3"
    assert shs.SystemPromptCache.try_load(tmp_path / "mini.shkv", m) is None


def test_shkv_truncated_inside_the_token_array_is_a_miss(shs, tmp_path):
    """TryLoad returns null on EndOfStreamException (SystemPromptCache.cs:140-164), also
    when the cut falls inside a token."""
    m = _FakeModel(shs)
    toks = np.arange(10, dtype=np.int32)
    c = shs.SystemPromptCache(toks, np.zeros(8, np.float32), shs.SystemPromptCache.compute_fingerprint(m, toks))
    c.save(tmp_path / "t.shkv")
    raw = (tmp_path / "t.shkv").read_bytes()
    start = 8 + 1 + 64 + 4
    for cut in (start + 1, start + 6, start + 39):
        (tmp_path / "t.shkv").write_bytes(raw[:cut])
        assert shs.SystemPromptCache.try_load(tmp_path / "t.shkv", m) is None

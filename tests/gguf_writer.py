"""Minimal GGUF v3 writer for test models (the container layout GgufFile.cs:110-199 reads)."""
import struct

import numpy as np

U32, I32, F32, STR, ARR = 4, 5, 6, 8, 9


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def yarn_keys(arch, cfg):
    """The rope.scaling.* and attention.temperature_scale keys the reference's converter
    writes for a YaRN checkpoint (tools/convert_shieldstral_to_gguf.py:307-323), from an
    oracle config's fields."""
    return [(f"{arch}.rope.scaling.type", STR, "yarn"),
            (f"{arch}.rope.scaling.factor", F32, cfg.rope_scale),
            (f"{arch}.rope.scaling.original_context_length", U32, cfg.rope_orig_ctx),
            (f"{arch}.rope.scaling.yarn_beta_fast", F32, cfg.yarn_beta_fast),
            (f"{arch}.rope.scaling.yarn_beta_slow", F32, cfg.yarn_beta_slow),
            (f"{arch}.rope.scaling.yarn_ext_factor", F32, cfg.yarn_ext_factor),
            (f"{arch}.rope.scaling.mscale", F32, cfg.yarn_mscale),
            (f"{arch}.rope.scaling.yarn_log_multiplier", F32, cfg.yarn_mscale_all_dim),
            (f"{arch}.rope.scaling.attn_factor", F32, cfg.rope_attn_factor),
            (f"{arch}.attention.temperature_scale", F32, cfg.attn_temperature),
            (f"{arch}.attention.temperature_length", U32, cfg.rope_orig_ctx)]


def write_gguf(path, arch, cfg, tensors, types, vocab_tokens=None, alignment=32, truncate_by=0, extra_kv=(),
               alignment_kv=None, offset_override=None):
    """cfg: the oracle/shs config fields; tensors: name → bytes/array; types: name → ggml id.
    extra_kv: more (key, type, value) entries; alignment_kv: the general.alignment entry's
    (type, value) when it should differ from the layout's alignment; offset_override:
    name → tensor offset written into the table instead of the real one."""
    kv = [("general.architecture", STR, arch),
          ("general.alignment",) + (alignment_kv or (U32, alignment)),
          (f"{arch}.block_count", U32, cfg.n_layer),
          (f"{arch}.embedding_length", U32, cfg.hidden),
          (f"{arch}.feed_forward_length", U32, cfg.ffn),
          (f"{arch}.attention.head_count", U32, cfg.n_head),
          (f"{arch}.attention.head_count_kv", U32, cfg.n_kv_head),
          (f"{arch}.attention.key_length", U32, cfg.head_dim),
          (f"{arch}.attention.layer_norm_rms_epsilon", F32, cfg.eps),
          (f"{arch}.rope.freq_base", F32, cfg.rope_theta),
          (f"{arch}.rope.dimension_count", U32, cfg.rope_dim)] + list(extra_kv)
    body = bytearray()
    for key, t, v in kv:
        body += _str(key) + struct.pack("<I", t)
        if t == STR:
            body += _str(v)
        elif t == U32:
            body += struct.pack("<I", v)
        elif t == F32:
            body += struct.pack("<f", v)
    n_kv = len(kv)
    toks = vocab_tokens if vocab_tokens is not None else [f"t{i}" for i in range(cfg.vocab)]
    body += _str("tokenizer.ggml.tokens") + struct.pack("<I", ARR) + struct.pack("<IQ", STR, len(toks))
    for s in toks:
        body += _str(s)
    n_kv += 1

    infos = bytearray()
    blobs = [(name, types[name], np.ascontiguousarray(data).tobytes()) for name, data in tensors.items()]
    off = 0
    q, kv_ = cfg.n_head * cfg.head_dim, cfg.n_kv_head * cfg.head_dim
    table = {"token_embd.weight": (cfg.hidden, cfg.vocab), "output_norm.weight": (cfg.hidden,)}
    for l in range(cfg.n_layer):
        p = f"blk.{l}."
        table.update({p + "attn_norm.weight": (cfg.hidden,), p + "ffn_norm.weight": (cfg.hidden,),
                      p + "attn_q.weight": (cfg.hidden, q), p + "attn_k.weight": (cfg.hidden, kv_),
                      p + "attn_v.weight": (cfg.hidden, kv_), p + "attn_output.weight": (q, cfg.hidden),
                      p + "ffn_gate.weight": (cfg.hidden, cfg.ffn), p + "ffn_up.weight": (cfg.hidden, cfg.ffn),
                      p + "ffn_down.weight": (cfg.ffn, cfg.hidden)})
    for name, t, raw in blobs:
        dims = table[name]
        infos += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        infos += struct.pack("<IQ", t, (offset_override or {}).get(name, off))
        off += len(raw)
        off = (off + alignment - 1) // alignment * alignment
    header = struct.pack("<IIQQ", 0x46554747, 3, len(blobs), n_kv)
    head = header + bytes(body) + bytes(infos)
    pad = (-len(head)) % alignment
    out = bytearray(head + b"\0" * pad)
    for name, t, raw in blobs:
        out += raw
        out += b"\0" * ((-len(raw)) % alignment)
    if truncate_by:
        out = out[:-truncate_by]
    with open(path, "wb") as f:
        f.write(out)

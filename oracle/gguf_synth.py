"""A GGUF v3 image of a synthetic BitNet-b1.58 model, and a state file of a
KV-cache prefix -- TEST INFRASTRUCTURE.

Packs the arrays of a model dict (saphira_llm_amd.synth_model) into the
container the reference loads (FORMAT.md:9-117 there): header, metadata,
tensor table, 32-byte-aligned data. The keys and tensor names are the ones
src/forward.c:318-455 reads; I2_S tensors carry n/4 + 32 bytes
(src/gguf.c:268-282), F16 / F32 their element size. Used only to hand the
same model to the reference's own sllm_model_load / sllm_forward.
"""
from __future__ import annotations

import struct

import numpy as np

GGUF_MAGIC = b"GGUF"
TYPE_U32, TYPE_F32, TYPE_STRING = 4, 6, 8
T_F32, T_F16, T_I2S = 0, 1, 36
ALIGN = 32

_NAMES = {"wq": "attn_q", "wk": "attn_k", "wv": "attn_v", "wo": "attn_output",
          "w_gate": "ffn_gate", "w_up": "ffn_up", "w_down": "ffn_down",
          "attn_norm": "attn_norm", "attn_sub_norm": "attn_sub_norm",
          "ffn_norm": "ffn_norm", "ffn_sub_norm": "ffn_sub_norm"}


def _str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _kv(key, vtype, value):
    out = _str(key) + struct.pack("<I", vtype)
    if vtype == TYPE_U32:
        return out + struct.pack("<I", value)
    if vtype == TYPE_F32:
        return out + struct.pack("<f", value)
    return out + _str(value)


def gguf_image(model, ctx_train=4096):
    """bytes of a GGUF file holding `model`."""
    cfg = model["cfg"]
    e, f, v = cfg["n_embd"], cfg["n_ff"], cfg["n_vocab"]
    gqa = e // cfg["n_head"] * cfg["n_head_kv"]
    arch = "bitnet-b1.58"
    kvs = [
        _kv("general.architecture", TYPE_STRING, arch),
        _kv(arch + ".block_count", TYPE_U32, cfg["n_layer"]),
        _kv(arch + ".embedding_length", TYPE_U32, e),
        _kv(arch + ".feed_forward_length", TYPE_U32, f),
        _kv(arch + ".attention.head_count", TYPE_U32, cfg["n_head"]),
        _kv(arch + ".attention.head_count_kv", TYPE_U32, cfg["n_head_kv"]),
        _kv(arch + ".rope.dimension_count", TYPE_U32, cfg["n_rot"]),
        _kv(arch + ".context_length", TYPE_U32, ctx_train),
        _kv(arch + ".vocab_size", TYPE_U32, v),
        _kv(arch + ".attention.layer_norm_rms_epsilon", TYPE_F32, cfg["eps"]),
        _kv(arch + ".rope.freq_base", TYPE_F32, cfg["rope_base"]),
    ]
    # (name, dims (ne0 first), type, bytes)
    tensors = [("token_embd.weight", (e, v), T_F16, np.ascontiguousarray(model["tok_embd"]).tobytes()),
               ("output_norm.weight", (e,), T_F32, np.ascontiguousarray(model["output_norm"]).tobytes())]
    dims = {"wq": (e, e), "wk": (e, gqa), "wv": (e, gqa), "wo": (e, e), "w_gate": (e, f),
            "w_up": (e, f), "w_down": (f, e), "attn_norm": (e,), "attn_sub_norm": (e,),
            "ffn_norm": (e,), "ffn_sub_norm": (f,)}
    for il, layer in enumerate(model["layers"]):
        for key, arr in layer.items():
            ttype = T_I2S if key.startswith("w") else T_F32
            tensors.append((f"blk.{il}.{_NAMES[key]}.weight", dims[key], ttype,
                            np.ascontiguousarray(arr).tobytes()))
    head = GGUF_MAGIC + struct.pack("<IQQ", 3, len(tensors), len(kvs)) + b"".join(kvs)
    table, blobs, offset = [], [], 0
    for name, d, ttype, data in tensors:
        table.append(_str(name) + struct.pack("<I", len(d)) + b"".join(struct.pack("<Q", x) for x in d)
                     + struct.pack("<IQ", ttype, offset))
        pad = (-len(data)) % ALIGN
        blobs.append(data + b"\0" * pad)
        offset += len(data) + pad
    meta = head + b"".join(table)
    meta += b"\0" * ((-len(meta)) % ALIGN)
    return meta + b"".join(blobs)


STATE_MAGIC, STATE_VERSION = 0x564B4C53, 1


def state_image(cfg, n_ctx, k, v, logits):
    """bytes of a state file in the layout src/forward.c:963-1036 reads and
    writes: magic, version, n_layer, n_ctx, n_head_kv, head dim, n_past,
    n_vocab, then per layer and KV head the live K rows then the live V rows,
    then the last position's logits. k / v: [n_layer][n_head_kv][n_past][hd]."""
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    n_layer, n_kv, n_past, hd = k.shape
    head = struct.pack("<IIiiiiii", STATE_MAGIC, STATE_VERSION, n_layer, n_ctx, n_kv, hd, n_past,
                       cfg["n_vocab"])
    body = b"".join(k[il, h].tobytes() + v[il, h].tobytes() for il in range(n_layer) for h in range(n_kv))
    return head + body + np.ascontiguousarray(logits, np.float32).tobytes()

"""ctypes access to the oracle libraries -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module, and only to check GPU results (or for the CPU figure
beside the GPU); the product path never does.

  liboracle.so          the C restatement (sllm_oracle.c), always built
  _ref/libsllm_ref.so   the reference's own hot-path sources compiled where
                        they lie (src/{status,log,isa,i2s_gemm,quant,thread,
                        topology}.c) plus ref_driver.c; present only when the
                        reference tree was available at build time
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_float, c_int, c_int32, c_size_t, c_uint8, c_uint64, c_void_p

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libsllm_ref.so")
# the same reference sources with src/forward.c patched to install the gfx950
# row (gfx950_forward.patch): the reference's own forward pass, GEMVs on the GPU
REF_GFX950_PATH = os.path.join(HERE, "_ref", "libsllm_ref_gfx950.so")

DOT_SCALAR, DOT_V3, DOT_VNNI = 0, 1, 2


class Act(ctypes.Structure):
    _fields_ = [("scale", c_float), ("sum", c_int32)]


_PROTOS = {
    "orc_quant_act": (None, [c_void_p, c_size_t, c_void_p, POINTER(Act)]),
    "orc_quant_act_rows": (None, [c_void_p, c_size_t, c_size_t, c_void_p, c_void_p]),
    "orc_dot_scalar": (c_int32, [c_void_p, c_void_p, c_size_t]),
    "orc_dot_v3": (c_int32, [c_void_p, c_void_p, c_size_t]),
    "orc_dot_vnni": (c_int32, [c_void_p, c_void_p, c_size_t]),
    "orc_vnni_supported": (c_int, []),
    "orc_gemv": (None, [c_void_p, c_size_t, c_size_t, c_void_p, c_void_p, c_int]),
    "orc_epilogue": (c_float, [c_int32, c_int32, c_float, c_float]),
    "orc_code": (c_uint8, [c_void_p, c_size_t]),
    "orc_scale": (c_float, [c_void_p, c_size_t]),
    "orc_dequant": (None, [c_void_p, c_void_p, c_size_t]),
    "orc_pack_converter": (None, [c_void_p, c_void_p, c_size_t]),
    "orc_linear": (None, [c_void_p, c_size_t, c_size_t, c_void_p, c_void_p, c_void_p, c_void_p,
                          POINTER(Act), c_int]),
    "orc_pool_create": (c_void_p, [c_int]),
    "orc_pool_destroy": (None, [c_void_p]),
    "orc_pool_threads": (c_int, [c_void_p]),
    "orc_gemv_parallel": (None, [c_void_p, c_void_p, c_size_t, c_size_t, c_void_p, c_void_p, c_int]),
    "orc_gemv_epilogue_parallel": (None, [c_void_p, c_void_p, c_size_t, c_size_t, c_void_p,
                                          POINTER(Act), c_void_p, c_void_p, c_int]),
    "orc_fnv1a64": (c_uint64, [c_void_p, c_size_t]),
    "orc_f16_to_f32": (c_float, [ctypes.c_uint16]),
    "orc_f16_to_f32_embd": (c_float, [ctypes.c_uint16]),
    "orc_rms_norm": (None, [c_void_p, c_void_p, c_void_p, c_size_t, c_float]),
    "orc_v_expf": (c_float, [c_float]),
    "orc_softmax": (None, [c_void_p, c_size_t]),
    "orc_silu": (None, [c_void_p, c_size_t]),
    "orc_rope_neox": (None, [c_void_p, c_size_t, c_int32, c_float, c_float]),
    "orc_rope_cos_sin": (None, [c_size_t, c_int32, c_float, c_float, c_void_p, c_void_p]),
    "orc_dot_f16": (c_float, [c_void_p, c_void_p, c_size_t]),
    "orc_argmax": (c_int32, [c_void_p, c_int32]),
    "orc_ctx_new": (c_void_p, [c_void_p, c_int32]),
    "orc_ctx_free": (None, [c_void_p]),
    "orc_ctx_k_cache": (c_void_p, [c_void_p]),
    "orc_ctx_v_cache": (c_void_p, [c_void_p]),
    "orc_forward_token": (c_int, [c_void_p, c_void_p, c_int32, c_int32, c_void_p, c_int, c_void_p, c_void_p]),
}

_REF_PROTOS = {
    "sllm_i2s_quant_act": (None, [c_void_p, c_size_t, c_void_p, POINTER(Act)]),
    "sllm_i2s_dot_scalar": (c_int32, [c_void_p, c_void_p, c_size_t]),
    "sllm_i2s_dot": (c_int32, [c_void_p, c_void_p, c_size_t]),
    "sllm_i2s_gemv": (None, [c_void_p, c_size_t, c_size_t, c_void_p, c_void_p]),
    "sllm_i2s_epilogue": (c_float, [c_int32, c_int32, c_float, c_float]),
    "sllm_i2s_select_level": (None, [c_int]),
    "sllm_i2s_select_auto": (None, []),
    "sllm_i2s_dot_isa": (c_int, []),
    "sllm_i2s_code": (c_uint8, [c_void_p, c_size_t]),
    "sllm_i2s_scale": (c_float, [c_void_p, c_size_t]),
    "sllm_i2s_dequant": (None, [c_void_p, c_void_p, c_size_t]),
    "ref_pool_create": (c_void_p, [c_int]),
    "sllm_pool_destroy": (None, [c_void_p]),
    "sllm_pool_threads": (c_int, [c_void_p]),
    "ref_gemv": (None, [c_void_p, c_void_p, c_size_t, c_size_t, c_void_p, c_void_p]),
    "ref_gemv_all": (None, [c_void_p, c_void_p, c_size_t, c_size_t, c_void_p, c_void_p]),
    "ref_gemv_epilogue": (None, [c_void_p, c_void_p, c_size_t, c_size_t, c_void_p, POINTER(Act),
                                 c_void_p, c_void_p, c_int]),
    "sllm_rms_norm": (None, [c_void_p, c_void_p, c_void_p, c_size_t, c_float]),
    "sllm_softmax_inplace": (None, [c_void_p, c_size_t]),
    "sllm_silu_inplace": (None, [c_void_p, c_size_t]),
    "sllm_rope_inplace": (None, [c_void_p, c_size_t, c_int32, c_float, c_float, c_int]),
    "sllm_dot_f16_f32": (c_float, [c_void_p, c_void_p, c_size_t]),
    "ref_model_open": (c_void_p, [c_void_p, c_size_t, POINTER(c_int)]),
    "ref_model_close": (None, [c_void_p]),
    "ref_ctx_new": (c_void_p, [c_void_p, c_int32]),
    "ref_ctx_free": (None, [c_void_p]),
    "ref_ctx_set_pool": (None, [c_void_p, c_void_p]),
    "ref_forward": (c_int, [c_void_p, c_void_p, c_int32, c_int32, c_void_p]),
    "ref_argmax": (c_int32, [c_void_p, c_int32]),
    "ref_state_load": (c_int, [c_void_p, c_void_p, ctypes.c_char_p]),
    "ref_forward_chunk": (c_int, [c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_void_p]),
    "ref_prefill_chunked": (c_int, [c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_void_p]),
}

# the reference's ISA levels as passed to sllm_i2s_select_level
# (include/saphira_llm/isa.h:35-42 orders V3 below VNNI)
_orc = None
_ref = None
_ref_gfx950 = None


def _bind(path, protos):
    lib = ctypes.CDLL(path)
    for name, (res, args) in protos.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def orc():
    global _orc
    if _orc is None:
        if not os.path.exists(ORACLE_PATH):
            raise ImportError(f"{ORACLE_PATH} not built: run `make -C {HERE}`")
        _orc = _bind(ORACLE_PATH, _PROTOS)
    return _orc


def ref_available():
    return os.path.exists(REF_PATH)


def ref():
    global _ref
    if _ref is None:
        _ref = _bind(REF_PATH, _REF_PROTOS)
    return _ref


def ref_gfx950_available():
    return os.path.exists(REF_GFX950_PATH)


def ref_gfx950():
    """The patched reference build (needs a gfx950 device to load a model)."""
    global _ref_gfx950
    if _ref_gfx950 is None:
        _ref_gfx950 = _bind(REF_GFX950_PATH, _REF_PROTOS)
    return _ref_gfx950


def _p(a):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(c_void_p)


# ---------------------------------------------------------------------------
# numpy-facing helpers
# ---------------------------------------------------------------------------

def quant_act(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    q = np.empty(x.size, dtype=np.int8)
    a = Act()
    orc().orc_quant_act(_p(x), x.size, _p(q), ctypes.byref(a))
    return q, np.float32(a.scale), int(a.sum)


def quant_act_rows(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    m, n = x.shape
    q = np.empty((m, n), dtype=np.int8)
    acts = (Act * m)()
    orc().orc_quant_act_rows(_p(x), n, m, _p(q), acts)
    return q, np.array([a.scale for a in acts], np.float32), np.array([a.sum for a in acts], np.int32)


def gemv(w, n_rows, n, q, path=DOT_V3):
    out = np.empty(n_rows, dtype=np.int32)
    orc().orc_gemv(_p(w), n_rows, n, _p(np.ascontiguousarray(q, np.int8)), _p(out), path)
    return out


def dot(w, q, n, path=DOT_SCALAR):
    fn = {DOT_SCALAR: orc().orc_dot_scalar, DOT_V3: orc().orc_dot_v3, DOT_VNNI: orc().orc_dot_vnni}[path]
    return int(fn(_p(w), _p(np.ascontiguousarray(q, np.int8)), n))


def epilogue(dot_, act_sum, act_scale, w_scale):
    return np.float32(orc().orc_epilogue(int(dot_), int(act_sum), float(act_scale), float(w_scale)))


def epilogue_rows(dots, act_sum, act_scale, w_scale):
    """The epilogue over an int32 row vector, one oracle call per element."""
    f = orc().orc_epilogue
    return np.array([f(int(d), int(act_sum), float(act_scale), float(w_scale)) for d in dots], np.float32)


def epilogue_np(dots, act_sum, act_scale, w_scale):
    """Vectorised restatement of src/i2s_gemm.c:271-290 in float32 numpy.

    post = w_scale / act_scale once (IEEE f32 division), then
    (float)(dot - act_sum) * post per element; checked against epilogue()
    in tests/test_oracle.py."""
    with np.errstate(divide="ignore", invalid="ignore"):
        post = np.float32(w_scale) / np.float32(act_scale)
        return (np.asarray(dots, np.int64) - int(act_sum)).astype(np.float32) * post


def scale(packed, n_elements):
    return np.float32(orc().orc_scale(_p(packed), n_elements))


def codes(packed, n):
    """Codes of elements 0..n-1 via orc_code."""
    f = orc().orc_code
    p = _p(packed)
    return np.array([f(p, k) for k in range(n)], np.uint8)


def dequant(packed, n):
    out = np.empty(n, np.float32)
    orc().orc_dequant(_p(packed), _p(out), n)
    return out


def pack_converter(codes_):
    codes_ = np.ascontiguousarray(codes_, np.uint8)
    n = codes_.size
    out = np.empty(n // 4 + 32, np.uint8)
    orc().orc_pack_converter(_p(out), _p(codes_), n)
    return out


def linear(w, n_rows, n, x, path=DOT_V3):
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(n_rows, np.float32)
    q = np.empty(n, np.int8)
    d = np.empty(n_rows, np.int32)
    a = Act()
    orc().orc_linear(_p(w), n_rows, n, _p(x), _p(y), _p(q), _p(d), ctypes.byref(a), path)
    return y, q, d, np.float32(a.scale), int(a.sum)


def fnv1a64(arr):
    arr = np.ascontiguousarray(arr)
    return int(orc().orc_fnv1a64(_p(arr), arr.nbytes))


class Pool:
    def __init__(self, threads):
        self.p = orc().orc_pool_create(threads)
        self.threads = orc().orc_pool_threads(self.p)

    def gemv(self, w, n_rows, n, q, out, path):
        orc().orc_gemv_parallel(self.p, _p(w), n_rows, n, _p(q), _p(out), path)

    def close(self):
        if self.p:
            orc().orc_pool_destroy(self.p)
            self.p = None


def lcg_activation(n):
    """The reference's fixed activation generator (tests/test_i2s.c:253-264,
    tools/reference/capture_i2s_golden.c:119-123): rng = 0xBEEF01;
    rng = rng*1664525 + 1013904223 (mod 2^32); x = (((rng>>8)&0xffff)/32768 - 1)*3
    evaluated in float32."""
    out = np.empty(n, np.float32)
    rng = 0xBEEF01
    for i in range(n):
        rng = (rng * 1664525 + 1013904223) & 0xFFFFFFFF
        v = np.float32((rng >> 8) & 0xFFFF) / np.float32(32768.0)
        out[i] = (np.float32(v) - np.float32(1.0)) * np.float32(3.0)
    return out


# ---------------------------------------------------------------------------
# the decode step
# ---------------------------------------------------------------------------

class OrcLayer(ctypes.Structure):
    """orc_layer"""
    _fields_ = [(n, c_void_p) for n in ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down",
                                         "attn_norm", "attn_sub_norm", "ffn_norm", "ffn_sub_norm")]


class OrcModel(ctypes.Structure):
    """orc_model"""
    _fields_ = [("n_layer", c_int32), ("n_embd", c_int32), ("n_ff", c_int32), ("n_head", c_int32),
                ("n_head_kv", c_int32), ("n_rot", c_int32), ("n_vocab", c_int32), ("eps", c_float),
                ("rope_base", c_float), ("tok_embd", c_void_p), ("output_norm", c_void_p),
                ("layers", c_void_p)]


def n_trace_dots(cfg):
    """int32 dots per token in a decode trace: per layer q, k, v, o, gate, up, down."""
    gqa = cfg["n_embd"] // cfg["n_head"] * cfg["n_head_kv"]
    return cfg["n_layer"] * (3 * cfg["n_embd"] + 2 * gqa + 2 * cfg["n_ff"])


class Decoder:
    """The oracle's decode step over a model dict (saphira_llm_amd.synth_model);
    keeps the numpy arrays alive for the C structs that point into them."""

    LAYER_KEYS = ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down",
                  "attn_norm", "attn_sub_norm", "ffn_norm", "ffn_sub_norm")

    def __init__(self, model, n_ctx):
        cfg = model["cfg"]
        self.model, self.cfg, self.n_ctx = model, cfg, n_ctx
        self.layers = (OrcLayer * cfg["n_layer"])()
        for il, layer in enumerate(model["layers"]):
            for k in self.LAYER_KEYS:
                setattr(self.layers[il], k, _p(layer[k]).value)
        self.m = OrcModel(cfg["n_layer"], cfg["n_embd"], cfg["n_ff"], cfg["n_head"], cfg["n_head_kv"],
                          cfg["n_rot"], cfg["n_vocab"], cfg["eps"], cfg["rope_base"],
                          _p(model["tok_embd"]).value, _p(model["output_norm"]).value,
                          ctypes.cast(self.layers, c_void_p).value)
        self.c = orc().orc_ctx_new(ctypes.byref(self.m), n_ctx)
        if not self.c:
            raise MemoryError("orc_ctx_new")
        hd = cfg["n_embd"] // cfg["n_head"]
        self.kv_shape = (cfg["n_layer"], cfg["n_head_kv"], n_ctx, hd)
        self.n_dots = n_trace_dots(cfg)

    def caches(self):
        """numpy views of the f32 K and V caches [layer][head_kv][pos][head_dim]."""
        n = int(np.prod(self.kv_shape))
        k = np.ctypeslib.as_array(ctypes.cast(orc().orc_ctx_k_cache(self.c), POINTER(c_float)), shape=(n,))
        v = np.ctypeslib.as_array(ctypes.cast(orc().orc_ctx_v_cache(self.c), POINTER(c_float)), shape=(n,))
        return k.reshape(self.kv_shape), v.reshape(self.kv_shape)

    def forward(self, token, pos, lm_threads=8, trace=False):
        """logits (and, with trace, every projection's int32 dots and every
        activation's (scale, sum)) of one token at position pos."""
        logits = np.empty(self.cfg["n_vocab"], np.float32)
        dots = np.empty(self.n_dots, np.int32) if trace else None
        acts = (Act * (4 * self.cfg["n_layer"]))() if trace else None
        st = orc().orc_forward_token(ctypes.byref(self.m), self.c, token, pos, _p(logits), lm_threads,
                                     _p(dots) if trace else None, acts)
        if st != 0:
            raise ValueError(f"orc_forward_token: bad token {token} or position {pos}")
        if not trace:
            return logits
        return logits, dots, np.array([(a.scale, a.sum) for a in acts],
                                      dtype=[("scale", "<f4"), ("sum", "<i4")])

    def close(self):
        if self.c:
            orc().orc_ctx_free(self.c)
            self.c = None


class RefDecoder:
    """The reference's own sllm_forward (oracle/_ref) on a GGUF image of the
    same model."""

    def __init__(self, model, n_ctx, threads=1, lib=None):
        from oracle.gguf_synth import gguf_image
        self.lib = lib if lib is not None else ref()
        self.image = np.frombuffer(gguf_image(model), np.uint8)
        st = c_int()
        self.r = self.lib.ref_model_open(_p(self.image), self.image.nbytes, ctypes.byref(st))
        if not self.r:
            raise ValueError(f"ref_model_open: status {st.value}")
        self.c = self.lib.ref_ctx_new(self.r, n_ctx)
        self.pool = self.lib.ref_pool_create(threads) if threads > 1 else None
        if self.pool:
            self.lib.ref_ctx_set_pool(self.c, self.pool)
        self.n_vocab = model["cfg"]["n_vocab"]

    def state_load(self, path):
        """sllm_state_load: the cache prefix and last logits from a state file."""
        st = self.lib.ref_state_load(self.r, self.c, path.encode())
        if st != 0:
            raise ValueError(f"sllm_state_load: status {st}")

    def forward(self, token, pos):
        logits = np.empty(self.n_vocab, np.float32)
        st = self.lib.ref_forward(self.r, self.c, token, pos, _p(logits))
        if st != 0:
            raise ValueError(f"sllm_forward: status {st}")
        return logits

    def forward_chunk(self, tokens, base):
        """sllm_forward_chunk: logits [n][n_vocab] of n tokens at base.."""
        t = np.ascontiguousarray(tokens, np.int32)
        logits = np.empty((t.size, self.n_vocab), np.float32)
        st = self.lib.ref_forward_chunk(self.r, self.c, _p(t), t.size, base, _p(logits))
        if st != 0:
            raise ValueError(f"sllm_forward_chunk: status {st}")
        return logits

    def prefill_chunked(self, tokens, chunk):
        """sllm_forward_prefill_chunked: logits [n][n_vocab]."""
        t = np.ascontiguousarray(tokens, np.int32)
        logits = np.empty((t.size, self.n_vocab), np.float32)
        st = self.lib.ref_prefill_chunked(self.r, self.c, _p(t), t.size, chunk, _p(logits))
        if st != 0:
            raise ValueError(f"sllm_forward_prefill_chunked: status {st}")
        return logits

    def close(self):
        if self.c:
            self.lib.ref_ctx_free(self.c)
            self.c = None
        if self.pool:
            self.lib.sllm_pool_destroy(self.pool)
            self.pool = None
        if self.r:
            self.lib.ref_model_close(self.r)
            self.r = None

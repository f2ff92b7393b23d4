"""ctypes bindings for libsllm_gfx950.so and libsllm_synth.so.

The product is the C ABI in include/saphira_amd/*.h; this module is the
plumbing the tests and bench.py use to reach it from Python. It holds no
compute of its own: every kernel call goes through the shared library, and
loading fails loudly (ImportError / GFX950Error) when the library is missing
or the device cannot be opened.

The directory name carries a hyphen, so load it by path::

    spec = importlib.util.spec_from_file_location("saphira_llm_amd", ".../__init__.py")
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_float, c_int, c_int32, c_size_t, c_uint, c_uint64, c_void_p

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libsllm_gfx950.so")
SYNTH_PATH = os.path.join(HERE, "libsllm_synth.so")

QK = 128
MAX_K = 65536
STATUS = {
    0: "ok", -1: "invalid-argument", -2: "out-of-memory", -4: "unsupported",
    -34: "wrong-tensor-shape", -36: "exceeds-limit", -60: "no-gfx950-device",
    -61: "hip-error", -62: "tensor-not-registered",
}


class Act(ctypes.Structure):
    """sllm_gfx950_act: layout of the reference's sllm_i2s_act."""
    _fields_ = [("scale", c_float), ("sum", c_int32)]


class GemvJob(ctypes.Structure):
    """sllm_gfx950_gemv_job."""
    _fields_ = [("w", c_void_p), ("n_rows", c_size_t), ("n", c_size_t), ("x", c_void_p),
                ("q", c_void_p), ("act", c_void_p), ("out", c_void_p), ("rows_out", c_void_p)]


class KernelRow(ctypes.Structure):
    """sllm_kernel_row."""
    _fields_ = [("name", c_char_p), ("priority", c_int),
                ("open", ctypes.CFUNCTYPE(c_int)),
                ("quant_act", ctypes.CFUNCTYPE(None, c_void_p, c_size_t, c_void_p, c_void_p)),
                ("dot", ctypes.CFUNCTYPE(c_int32, c_void_p, c_void_p, c_size_t)),
                ("gemv", ctypes.CFUNCTYPE(None, c_void_p, c_size_t, c_size_t, c_void_p, c_void_p)),
                ("release", ctypes.CFUNCTYPE(None))]


class LayerDesc(ctypes.Structure):
    """sllm_gfx950_layer_desc: one block's host tensors."""
    _fields_ = [(n, c_void_p) for n in ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down",
                                        "attn_norm", "attn_sub_norm", "ffn_norm", "ffn_sub_norm")]


class GemmJob(ctypes.Structure):
    """sllm_gfx950_gemm_job: one tensor of a multi-tensor GEMM."""
    _fields_ = [("w", c_void_p), ("n_rows", c_size_t), ("out", c_void_p), ("rows_out", c_void_p)]


class GemmPlanJob(ctypes.Structure):
    """sllm_gfx950_gemm_plan_job: one tensor of a GEMM plan."""
    _fields_ = [("w", c_void_p), ("n_rows", c_size_t), ("n", c_size_t), ("q", c_void_p),
                ("act", c_void_p), ("out", c_void_p), ("rows_out", c_void_p)]


class ModelDesc(ctypes.Structure):
    """sllm_gfx950_model_desc."""
    _fields_ = [("n_layer", c_int32), ("n_embd", c_int32), ("n_ff", c_int32), ("n_head", c_int32),
                ("n_head_kv", c_int32), ("n_rot", c_int32), ("n_vocab", c_int32),
                ("eps", c_float), ("rope_base", c_float),
                ("tok_embd", c_void_p), ("output_norm", c_void_p), ("layers", POINTER(LayerDesc))]


# Every function the C ABI exports: name -> (restype, argtypes).
PROTOTYPES = {
    "sllm_gfx950_open": (c_int, [c_int]),
    "sllm_gfx950_close": (None, []),
    "sllm_gfx950_is_open": (c_int, []),
    "sllm_gfx950_status_string": (c_char_p, [c_int]),
    "sllm_gfx950_last_error": (c_char_p, []),
    "sllm_gfx950_device_info": (c_int, [c_char_p, c_size_t, POINTER(c_int), POINTER(c_size_t)]),
    "sllm_gfx950_malloc": (c_int, [POINTER(c_void_p), c_size_t]),
    "sllm_gfx950_free": (c_int, [c_void_p]),
    "sllm_gfx950_h2d": (c_int, [c_void_p, c_void_p, c_size_t]),
    "sllm_gfx950_d2h": (c_int, [c_void_p, c_void_p, c_size_t]),
    "sllm_gfx950_sync": (c_int, []),
    "sllm_gfx950_stream": (c_void_p, []),
    "sllm_gfx950_timer_start": (c_int, []),
    "sllm_gfx950_timer_stop": (c_int, [POINTER(c_float)]),
    "sllm_gfx950_events_reserve": (c_int, [c_int]),
    "sllm_gfx950_event_record": (c_int, [c_int]),
    "sllm_gfx950_event_elapsed": (c_int, [c_int, c_int, POINTER(c_float)]),
    "sllm_gfx950_copy": (c_int, [c_void_p, c_void_p, c_size_t]),
    "sllm_gfx950_checksum": (c_int, [c_void_p, c_size_t, c_void_p, c_uint]),
    "sllm_gfx950_diag_expf": (c_int, [c_uint, c_uint, c_uint, c_void_p]),
    "sllm_gfx950_quant_act": (c_int, [c_void_p, c_size_t, c_size_t, c_void_p, c_void_p]),
    "sllm_gfx950_gemv": (c_int, [c_void_p, c_size_t, c_size_t, c_void_p, c_void_p]),
    "sllm_gfx950_gemv_epilogue": (c_int, [c_void_p, c_size_t, c_size_t, c_void_p, c_void_p, c_void_p]),
    "sllm_gfx950_linear": (c_int, [c_void_p, c_size_t, c_size_t, c_void_p, c_void_p, c_void_p, c_void_p]),
    "sllm_gfx950_gemv_batch": (c_int, [POINTER(GemvJob), c_size_t]),
    "sllm_gfx950_gemv_batch_noalloc": (c_int, [POINTER(GemvJob), c_size_t]),
    "sllm_gfx950_plan_create": (c_int, [POINTER(GemvJob), c_size_t, POINTER(c_void_p)]),
    "sllm_gfx950_plan_run": (c_int, [c_void_p]),
    "sllm_gfx950_plan_run_marked": (c_int, [c_void_p, c_int]),
    "sllm_gfx950_plan_destroy": (None, [c_void_p]),
    "sllm_gfx950_set_tuning": (c_int, [c_int, c_int, c_int, c_int, c_int, c_int]),
    "sllm_gfx950_tensor_register": (c_int, [c_void_p, c_size_t, c_size_t]),
    "sllm_gfx950_tensor_unregister": (c_int, [c_void_p]),
    "sllm_gfx950_tensor_acquire": (c_int, [c_void_p, c_size_t, c_size_t]),
    "sllm_gfx950_tensor_release_acquired": (c_int, []),
    "sllm_gfx950_tensor_device": (c_void_p, [c_void_p]),
    "sllm_gfx950_i2s_quant_act": (None, [c_void_p, c_size_t, c_void_p, c_void_p]),
    "sllm_gfx950_i2s_dot": (c_int32, [c_void_p, c_void_p, c_size_t]),
    "sllm_gfx950_i2s_gemv": (None, [c_void_p, c_size_t, c_size_t, c_void_p, c_void_p]),
    "sllm_kdispatch_register": (c_int, [POINTER(KernelRow)]),
    "sllm_kdispatch_count": (c_size_t, []),
    "sllm_kdispatch_row": (POINTER(KernelRow), [c_size_t]),
    "sllm_kdispatch_select": (c_int, [c_char_p]),
    "sllm_kdispatch_installed": (POINTER(KernelRow), []),
    "sllm_kdispatch_installed_name": (c_char_p, []),
    "sllm_kdispatch_reset": (None, []),
    "sllm_kdispatch_quant_act": (None, [c_void_p, c_size_t, c_void_p, c_void_p]),
    "sllm_kdispatch_dot": (c_int32, [c_void_p, c_void_p, c_size_t]),
    "sllm_kdispatch_gemv": (None, [c_void_p, c_size_t, c_size_t, c_void_p, c_void_p]),
    "sllm_kdispatch_release": (None, []),
    "sllm_gfx950_gemm": (c_int, [c_void_p, c_size_t, c_size_t, c_void_p, c_void_p, c_size_t, c_void_p, c_void_p]),
    "sllm_gfx950_linear_batch": (c_int, [c_void_p, c_size_t, c_size_t, c_void_p, c_size_t, c_void_p, c_void_p,
                                         c_void_p, c_void_p]),
    "sllm_gfx950_set_gemm_tile": (c_int, [c_int]),
    "sllm_gfx950_gemm_plan_create": (c_int, [POINTER(GemmPlanJob), c_size_t, c_size_t, POINTER(c_void_p)]),
    "sllm_gfx950_gemm_plan_run": (c_int, [c_void_p]),
    "sllm_gfx950_gemm_plan_destroy": (None, [c_void_p]),
    "sllm_gfx950_gemm_multi": (c_int, [c_void_p, c_size_t, c_size_t, c_void_p, c_void_p, c_size_t]),
    "sllm_gfx950_model_upload": (c_int, [POINTER(ModelDesc), POINTER(c_void_p)]),
    "sllm_gfx950_model_free": (None, [c_void_p]),
    "sllm_gfx950_model_load_gguf": (c_int, [c_void_p, c_size_t, POINTER(c_void_p)]),
    "sllm_gfx950_model_load_gguf_file": (c_int, [c_char_p, POINTER(c_void_p)]),
    "sllm_gfx950_gguf_describe": (c_int, [c_void_p, c_size_t, POINTER(ModelDesc), POINTER(LayerDesc)]),
    "sllm_gfx950_ctx_new": (c_int, [c_void_p, c_int32, POINTER(c_void_p)]),
    "sllm_gfx950_ctx_free": (None, [c_void_p]),
    "sllm_gfx950_ctx_reset": (c_int, [c_void_p]),
    "sllm_gfx950_ctx_n_past": (c_int32, [c_void_p]),
    "sllm_gfx950_forward": (c_int, [c_void_p, c_void_p, c_int32, c_int32, c_void_p]),
    "sllm_gfx950_generate_greedy": (c_int, [c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_void_p]),
    "sllm_gfx950_forward_chunk": (c_int, [c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_void_p]),
    "sllm_gfx950_forward_prefill_chunked": (c_int, [c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_void_p]),
    "sllm_gfx950_ctx_logits": (c_void_p, [c_void_p]),
    "sllm_gfx950_ctx_argmax": (c_int, [c_void_p, POINTER(c_int32)]),
    "sllm_gfx950_ctx_kv_load": (c_int, [c_void_p, c_void_p, c_void_p, c_int32, c_void_p]),
    "sllm_gfx950_ctx_set_inflight": (c_int, [c_void_p, c_int32]),
    "sllm_gfx950_ctx_set_graph": (c_int, [c_void_p, c_int]),
    "sllm_gfx950_trace_dots": (c_size_t, [c_void_p]),
    "sllm_gfx950_ctx_trace": (c_int, [c_void_p, c_void_p, c_void_p]),
}

SYNTH_PROTOTYPES = {
    "sllm_synth_seed": (c_uint64, [c_uint, c_uint, c_uint, c_uint]),
    "sllm_synth_scale": (c_float, [c_uint64]),
    "sllm_synth_codes": (None, [c_uint64, c_size_t, c_size_t, c_void_p]),
    "sllm_synth_i2s": (c_int, [c_uint64, c_size_t, c_size_t, c_void_p, c_int]),
    "sllm_synth_normal": (None, [c_uint64, c_size_t, c_void_p]),
    "sllm_synth_normal_f16": (None, [c_uint64, c_size_t, c_void_p, c_int]),
    "sllm_expf_mismatches": (c_uint64, [c_uint64, c_uint64, c_int, POINTER(ctypes.c_uint32)]),
    "sllm_expf_strided": (None, [c_uint, c_uint, c_uint64, c_void_p, c_int]),
}

_lib = None
_synth = None


def _bind(path, protos):
    if not os.path.exists(path):
        raise ImportError(f"{path} is not built: run `make -C {HERE}` (or __graft_entry__.build())")
    lib = ctypes.CDLL(path)
    for name, (res, args) in protos.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def lib():
    """The loaded libsllm_gfx950.so with every prototype set."""
    global _lib
    if _lib is None:
        _lib = _bind(LIB_PATH, PROTOTYPES)
    return _lib


def synth_lib():
    global _synth
    if _synth is None:
        _synth = _bind(SYNTH_PATH, SYNTH_PROTOTYPES)
    return _synth


class GFX950Error(RuntimeError):
    def __init__(self, status, where=""):
        msg = lib().sllm_gfx950_last_error().decode(errors="replace")
        super().__init__(f"{where}: {STATUS.get(status, status)} ({status}): {msg}")
        self.status = status


def check(status, where=""):
    if status != 0:
        raise GFX950Error(status, where)
    return status


def ptr(a):
    """Host address of a contiguous numpy array."""
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(c_void_p)


# ---------------------------------------------------------------------------
# device handle
# ---------------------------------------------------------------------------

class DevBuf:
    """A device allocation owned by the library (freed by free() or the Device)."""

    def __init__(self, dev, nbytes):
        self.dev = dev
        self.nbytes = int(nbytes)
        p = c_void_p()
        check(lib().sllm_gfx950_malloc(ctypes.byref(p), self.nbytes), "malloc")
        self.ptr = p.value

    def at(self, offset):
        return c_void_p(self.ptr + int(offset))

    @property
    def vp(self):
        return c_void_p(self.ptr)

    def upload(self, arr, offset=0):
        arr = np.ascontiguousarray(arr)
        assert offset + arr.nbytes <= self.nbytes
        check(lib().sllm_gfx950_h2d(self.at(offset), ptr(arr), arr.nbytes), "h2d")

    def download(self, dtype, count, offset=0):
        out = np.empty(count, dtype=dtype)
        assert offset + out.nbytes <= self.nbytes
        check(lib().sllm_gfx950_d2h(ptr(out), self.at(offset), out.nbytes), "d2h")
        return out

    def free(self):
        if self.ptr:
            check(lib().sllm_gfx950_free(c_void_p(self.ptr)), "free")
            self.ptr = 0


class Device:
    """sllm_gfx950_open on `device`; raises GFX950Error when there is no gfx950."""

    def __init__(self, device=0):
        self.lib = lib()
        check(self.lib.sllm_gfx950_open(device), "open")
        name = ctypes.create_string_buffer(520)
        cu, hbm = c_int(), c_size_t()
        check(self.lib.sllm_gfx950_device_info(name, 520, ctypes.byref(cu), ctypes.byref(hbm)), "info")
        self.name, self.cu, self.hbm = name.value.decode(), cu.value, hbm.value

    def alloc(self, nbytes):
        return DevBuf(self, nbytes)

    def put(self, arr):
        arr = np.ascontiguousarray(arr)
        b = DevBuf(self, max(arr.nbytes, 1))
        b.upload(arr)
        return b

    def sync(self):
        check(self.lib.sllm_gfx950_sync(), "sync")

    def timer_start(self):
        check(self.lib.sllm_gfx950_timer_start(), "timer_start")

    def timer_stop(self):
        ms = c_float()
        check(self.lib.sllm_gfx950_timer_stop(ctypes.byref(ms)), "timer_stop")
        return ms.value

    def events(self, n):
        check(self.lib.sllm_gfx950_events_reserve(n), "events_reserve")

    def record(self, i):
        check(self.lib.sllm_gfx950_event_record(i), "event_record")

    def elapsed(self, i, j):
        ms = c_float()
        check(self.lib.sllm_gfx950_event_elapsed(i, j, ctypes.byref(ms)), "event_elapsed")
        return ms.value

    def copy(self, dst, src, nbytes):
        check(self.lib.sllm_gfx950_copy(dst, src, nbytes), "copy")

    def checksum(self, src, nbytes, partials, n_partials):
        check(self.lib.sllm_gfx950_checksum(src, nbytes, partials, n_partials), "checksum")

    # device-pointer kernels -------------------------------------------------
    def quant_act(self, x, n, n_tok, q, act):
        check(self.lib.sllm_gfx950_quant_act(x, n, n_tok, q, act), "quant_act")

    def gemv(self, w, n_rows, n, q, rows_out):
        check(self.lib.sllm_gfx950_gemv(w, n_rows, n, q, rows_out), "gemv")

    def gemv_epilogue(self, w, n_rows, n, q, act, out):
        check(self.lib.sllm_gfx950_gemv_epilogue(w, n_rows, n, q, act, out), "gemv_epilogue")

    def linear(self, w, n_rows, n, x, q, act, out):
        check(self.lib.sllm_gfx950_linear(w, n_rows, n, x, q, act, out), "linear")

    def gemv_batch(self, jobs):
        arr = (GemvJob * len(jobs))(*jobs)
        check(self.lib.sllm_gfx950_gemv_batch(arr, len(jobs)), "gemv_batch")

    def gemv_batch_noalloc(self, jobs):
        arr = (GemvJob * len(jobs))(*jobs)
        check(self.lib.sllm_gfx950_gemv_batch_noalloc(arr, len(jobs)), "gemv_batch_noalloc")

    def plan(self, jobs):
        arr = (GemvJob * len(jobs))(*jobs)
        p = c_void_p()
        check(self.lib.sllm_gfx950_plan_create(arr, len(jobs), ctypes.byref(p)), "plan_create")
        return p

    def plan_run(self, p, event=None):
        if event is None:
            check(self.lib.sllm_gfx950_plan_run(p), "plan_run")
        else:
            check(self.lib.sllm_gfx950_plan_run_marked(p, event), "plan_run_marked")

    def plan_destroy(self, p):
        self.lib.sllm_gfx950_plan_destroy(p)

    def gemm(self, w, n_rows, n, q, act, m, out, rows_out=None):
        check(self.lib.sllm_gfx950_gemm(w, n_rows, n, q, act, m, out, rows_out), "gemm")

    def gemm_multi(self, jobs, n, q, act, m):
        """jobs: (w, n_rows, out, rows_out) device pointers per tensor (1 to 3)."""
        arr = (GemmJob * len(jobs))(*[GemmJob(w, n_rows, out, ro) for w, n_rows, out, ro in jobs])
        check(self.lib.sllm_gfx950_gemm_multi(arr, len(jobs), n, q, act, m), "gemm_multi")

    def linear_batch(self, w, n_rows, n, x, m, q, act, out, rows_out=None):
        check(self.lib.sllm_gfx950_linear_batch(w, n_rows, n, x, m, q, act, out, rows_out), "linear_batch")

    def gemm_plan(self, jobs, m):
        """A GEMM plan over (w, n_rows, k, q, act, out, rows_out) jobs of m tokens."""
        arr = (GemmPlanJob * len(jobs))(*[GemmPlanJob(*j) for j in jobs])
        p = ctypes.c_void_p()
        check(self.lib.sllm_gfx950_gemm_plan_create(arr, len(jobs), m, ctypes.byref(p)), "gemm_plan_create")
        return p

    def gemm_plan_run(self, p):
        check(self.lib.sllm_gfx950_gemm_plan_run(p), "gemm_plan_run")

    def gemm_plan_destroy(self, p):
        self.lib.sllm_gfx950_gemm_plan_destroy(p)

    def set_gemm_tile(self, tile=0):
        check(self.lib.sllm_gfx950_set_gemm_tile(tile), "set_gemm_tile")

    def set_tuning(self, path=0, variant=-1, lanes_per_row=0, waves=0, rows_per_wg=0, slab_kib=0):
        check(self.lib.sllm_gfx950_set_tuning(path, variant, lanes_per_row, waves, rows_per_wg, slab_kib),
              "set_tuning")


# ---------------------------------------------------------------------------
# synthetic workloads
# ---------------------------------------------------------------------------

def synth_seed(cfg, set_=0, layer=0, matrix=0):
    return synth_lib().sllm_synth_seed(cfg, set_, layer, matrix)


def synth_scale(seed):
    return np.float32(synth_lib().sllm_synth_scale(seed))


def synth_codes(seed, n_rows, n):
    out = np.empty(n_rows * n, dtype=np.uint8)
    synth_lib().sllm_synth_codes(seed, n_rows, n, ptr(out))
    return out.reshape(n_rows, n)


def synth_i2s(seed, n_rows, n, threads=None, out=None):
    """Packed tensor bytes (n_rows*n/4 + 32, uint8) for tensor `seed`."""
    if threads is None:
        threads = min(16, os.cpu_count() or 1)
    nbytes = n_rows * (n // 4) + 32
    if out is None:
        out = np.empty(nbytes, dtype=np.uint8)
    assert out.nbytes == nbytes and out.dtype == np.uint8
    if synth_lib().sllm_synth_i2s(seed, n_rows, n, ptr(out), threads) != 0:
        raise ValueError(f"synth_i2s: bad shape {n_rows}x{n}")
    return out


def synth_normal(seed, count):
    out = np.empty(count, dtype=np.float32)
    synth_lib().sllm_synth_normal(seed, count, ptr(out))
    return out


def synth_normal_f16(seed, count, threads=None):
    """synth_normal(seed, count) rounded to binary16, as uint16 bits."""
    if threads is None:
        threads = min(16, os.cpu_count() or 1)
    out = np.empty(count, dtype=np.uint16)
    synth_lib().sllm_synth_normal_f16(seed, count, ptr(out), threads)
    return out


# BitNet-b1.58-2B shapes (the reference's PHASE4 contract: 30 layers, n_embd
# 2560, n_ff 6912, 20 query heads of 128, 5 KV heads, vocab 128256, RoPE
# NeoX base 500000, eps 1e-5)
BITNET_2B = dict(n_layer=30, n_embd=2560, n_ff=6912, n_head=20, n_head_kv=5, n_rot=128,
                 n_vocab=128256, eps=1e-5, rope_base=500000.0)

LAYER_I2S = ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down")
LAYER_NORMS = ("attn_norm", "attn_sub_norm", "ffn_norm", "ffn_sub_norm")


def synth_model(cfg, seed_set=0, threads=None):
    """A random-init BitNet-b1.58 model of shape `cfg` (see BITNET_2B):
    uniform ternary I2_S projections with per-tensor scales U(0.5, 2), norm
    weights N(1, 0.1^2), an F16 N(0, 1) token embedding (also the lm_head).
    Returns {"cfg": cfg, "tok_embd": uint16[n_vocab * n_embd],
    "output_norm": f32[n_embd], "layers": [{name: array}]}; I2_S arrays are
    the packed bytes with their 32-byte tails."""
    e, f = cfg["n_embd"], cfg["n_ff"]
    gqa = e // cfg["n_head"] * cfg["n_head_kv"]
    shapes = {"wq": (e, e), "wk": (gqa, e), "wv": (gqa, e), "wo": (e, e),
              "w_gate": (f, e), "w_up": (f, e), "w_down": (e, f)}
    norm_len = {"attn_norm": e, "attn_sub_norm": e, "ffn_norm": e, "ffn_sub_norm": f}
    model = {"cfg": dict(cfg), "layers": []}
    model["tok_embd"] = synth_normal_f16(synth_seed(4, seed_set, 0, 900), cfg["n_vocab"] * e, threads)
    model["output_norm"] = (np.float32(1) + np.float32(0.1) * synth_normal(synth_seed(4, seed_set, 0, 901), e)).astype(np.float32)
    for il in range(cfg["n_layer"]):
        layer = {}
        for m, name in enumerate(LAYER_I2S):
            n_rows, n = shapes[name]
            layer[name] = synth_i2s(synth_seed(4, seed_set, il, m), n_rows, n, threads)
        for m, name in enumerate(LAYER_NORMS):
            layer[name] = (np.float32(1) + np.float32(0.1) * synth_normal(synth_seed(4, seed_set, il, 16 + m),
                                                                          norm_len[name])).astype(np.float32)
        model["layers"].append(layer)
    return model


def model_desc(model):
    """(ModelDesc, keep-alive list) describing a synth_model dict's host arrays."""
    cfg = model["cfg"]
    keep = []

    def p(a):
        a = np.ascontiguousarray(a)
        keep.append(a)
        return a.ctypes.data_as(c_void_p)

    layers = (LayerDesc * cfg["n_layer"])()
    for il, L in enumerate(model["layers"]):
        for name in LAYER_I2S + LAYER_NORMS:
            setattr(layers[il], name, p(L[name]))
    keep.append(layers)
    d = ModelDesc(cfg["n_layer"], cfg["n_embd"], cfg["n_ff"], cfg["n_head"], cfg["n_head_kv"], cfg["n_rot"],
                  cfg["n_vocab"], cfg["eps"], cfg["rope_base"], p(model["tok_embd"]), p(model["output_norm"]),
                  layers)
    return d, keep


GGUF_MAX_LAYERS = 64


def gguf_describe(image):
    """(status, cfg, tensors) of a GGUF image read by sllm_gfx950_gguf_describe
    (no device needed): cfg holds the hyper-parameters, tensors maps
    "tok_embd", "output_norm" and (layer, name) to the byte offset in the
    image where that tensor's data starts. cfg and tensors are None unless
    the status is 0."""
    n = len(image)
    buf = np.frombuffer(image, np.uint8) if n else np.zeros(1, np.uint8)
    d = ModelDesc()
    layers = (LayerDesc * GGUF_MAX_LAYERS)()
    st = lib().sllm_gfx950_gguf_describe(ptr(buf), n, ctypes.byref(d), layers)
    if st != 0:
        return st, None, None
    base = buf.ctypes.data
    cfg = {"n_layer": d.n_layer, "n_embd": d.n_embd, "n_ff": d.n_ff, "n_head": d.n_head,
           "n_head_kv": d.n_head_kv, "n_rot": d.n_rot, "n_vocab": d.n_vocab, "eps": d.eps,
           "rope_base": d.rope_base}
    tensors = {"tok_embd": d.tok_embd - base, "output_norm": d.output_norm - base}
    for il in range(d.n_layer):
        for name in LAYER_I2S + LAYER_NORMS:
            tensors[(il, name)] = getattr(layers[il], name) - base
    return st, cfg, tensors


class DeviceDecoder:
    """A model uploaded with sllm_gfx950_model_upload (or, gguf given, read
    from a GGUF image -- bytes -- or file -- a path -- with
    sllm_gfx950_model_load_gguf[_file]) and one context of n_ctx positions
    (sllm_gfx950_ctx_new): the decode step on the GPU."""

    def __init__(self, dev, model, n_ctx, gguf=None):
        self.dev = dev
        L = lib()
        m = c_void_p()
        if isinstance(gguf, (str, os.PathLike)):
            check(L.sllm_gfx950_model_load_gguf_file(os.fsencode(gguf), ctypes.byref(m)), "model_load_gguf_file")
            with open(gguf, "rb") as fh:
                self.cfg = gguf_describe(fh.read())[1]
        elif gguf is not None:
            buf = np.frombuffer(gguf, np.uint8)
            check(L.sllm_gfx950_model_load_gguf(ptr(buf), buf.size, ctypes.byref(m)), "model_load_gguf")
            self.cfg = gguf_describe(gguf)[1]
        else:
            self.cfg = dict(model["cfg"])
            d, keep = model_desc(model)
            check(L.sllm_gfx950_model_upload(ctypes.byref(d), ctypes.byref(m)), "model_upload")
            del keep
        self.m = m
        c = c_void_p()
        st = L.sllm_gfx950_ctx_new(m, n_ctx, ctypes.byref(c))
        if st != 0:
            L.sllm_gfx950_model_free(m)
            check(st, "ctx_new")
        self.c = c
        self.n_ctx = n_ctx

    def forward(self, token, pos, logits=True):
        """Logits (float32[n_vocab]) of `token` at `pos`, or None with logits=False."""
        out = np.empty(self.cfg["n_vocab"], np.float32) if logits else None
        check(lib().sllm_gfx950_forward(self.m, self.c, token, pos, ptr(out) if logits else None), "forward")
        return out

    def forward_chunk(self, tokens, base, logits=True):
        """Logits (float32[n][n_vocab]) of n tokens as one chunk at base.., or
        None with logits=False (the last token's stay on the device)."""
        t = np.ascontiguousarray(tokens, np.int32)
        out = np.empty((t.size, self.cfg["n_vocab"]), np.float32) if logits else None
        check(lib().sllm_gfx950_forward_chunk(self.m, self.c, ptr(t) if t.size else None, t.size, base,
                                              ptr(out) if logits else None), "forward_chunk")
        return out

    def status_chunk(self, tokens, base):
        """The raw status of a chunk forward without logits (argument checks)."""
        t = np.ascontiguousarray(tokens, np.int32)
        return lib().sllm_gfx950_forward_chunk(self.m, self.c, ptr(t) if t.size else None, t.size, base, None)

    def prefill_chunked(self, tokens, chunk, logits=True):
        t = np.ascontiguousarray(tokens, np.int32)
        out = np.empty((t.size, self.cfg["n_vocab"]), np.float32) if logits else None
        check(lib().sllm_gfx950_forward_prefill_chunked(self.m, self.c, ptr(t) if t.size else None, t.size, chunk,
                                                        ptr(out) if logits else None), "forward_prefill_chunked")
        return out

    def status_prefill(self, tokens, chunk):
        t = np.ascontiguousarray(tokens, np.int32)
        return lib().sllm_gfx950_forward_prefill_chunked(self.m, self.c, ptr(t) if t.size else None, t.size,
                                                         chunk, None)

    def status_forward(self, token, pos):
        """The raw status of a forward (for argument checks)."""
        return lib().sllm_gfx950_forward(self.m, self.c, token, pos, None)

    def argmax(self):
        t = c_int32()
        check(lib().sllm_gfx950_ctx_argmax(self.c, ctypes.byref(t)), "ctx_argmax")
        return t.value

    def generate(self, prompt, n_new):
        pr = np.ascontiguousarray(prompt, np.int32)
        out = np.zeros(max(n_new, 1), np.int32)
        check(lib().sllm_gfx950_generate_greedy(self.m, self.c, ptr(pr) if pr.size else None, pr.size, n_new,
                                                ptr(out)), "generate_greedy")
        return out[:n_new]

    def kv_load(self, k, v, n_pos, logits=None):
        """Restore a cache prefix of n_pos positions (k, v: [layer][head_kv]
        [n_pos][head_dim]) and, given, the last position's logits."""
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        lg = None if logits is None else np.ascontiguousarray(logits, np.float32)
        check(lib().sllm_gfx950_ctx_kv_load(self.c, ptr(k), ptr(v), n_pos, None if lg is None else ptr(lg)),
              "ctx_kv_load")

    def set_inflight(self, tokens):
        check(lib().sllm_gfx950_ctx_set_inflight(self.c, tokens), "ctx_set_inflight")

    def reset(self):
        check(lib().sllm_gfx950_ctx_reset(self.c), "ctx_reset")

    def n_past(self):
        return lib().sllm_gfx950_ctx_n_past(self.c)

    def set_graph(self, on):
        check(lib().sllm_gfx950_ctx_set_graph(self.c, 1 if on else 0), "ctx_set_graph")

    def trace_start(self):
        """Record every projection's dots and every activation's scale/sum."""
        n = lib().sllm_gfx950_trace_dots(self.m)
        self.t_dots = self.dev.alloc(4 * n)
        self.t_acts = self.dev.alloc(8 * 4 * self.cfg["n_layer"])
        self.t_n = n
        check(lib().sllm_gfx950_ctx_trace(self.c, self.t_dots.vp, self.t_acts.vp), "ctx_trace")

    def trace_read(self):
        self.dev.sync()
        dots = self.t_dots.download(np.int32, self.t_n)
        raw = self.t_acts.download(np.uint8, 8 * 4 * self.cfg["n_layer"])
        acts = np.frombuffer(raw.tobytes(), dtype=[("scale", "<f4"), ("sum", "<i4")])
        return dots, acts

    def trace_stop(self):
        check(lib().sllm_gfx950_ctx_trace(self.c, None, None), "ctx_trace")
        self.t_dots.free()
        self.t_acts.free()

    def close(self):
        if getattr(self, "c", None):
            lib().sllm_gfx950_ctx_free(self.c)
            self.c = None
        if getattr(self, "m", None):
            lib().sllm_gfx950_model_free(self.m)
            self.m = None

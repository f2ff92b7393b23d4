"""HIP failures on the host side, on the CPU.

The library's C sources linked against tests/fakehip/fake_hip.c (a
host-memory stand-in for the HIP runtime) make
tests/fakehip/libsllm_gfx950_fakehip.so: one fake gfx950 device, kernels
that do nothing, and any HIP call made to fail on demand. With it, every
status-returning device and decode entry point is driven through every HIP
call it makes, one failure at a time:

  * a failed hipMalloc / hipHostMalloc (out of memory) returns -2, the
    reference's SLLM_ERR_NOMEM (include/saphira_llm/status.h);
  * any other failed HIP call returns -61 (SLLM_GFX950_ERR_HIP);
  * either way nothing the call allocated is left behind, the message names
    the call, and the same call succeeds once nothing fails;
  * before sllm_gfx950_open, every entry point returns -60 (no device);
  * a failed hipModuleLoadData leaves the library closed and a later open
    works;
  * the host-pointer row (void / int32 signatures: no status to return)
    prints the reason and aborts, shown in a child process.

This is the library's counterpart of the reference's test that its gates can
fail (tests/test_gate_propagation.c): induced failures, not the absence of
failures, show that errors reach the caller.
"""
import ctypes
import os
import subprocess
import sys
from ctypes import byref, c_char_p, c_float, c_int, c_int32, c_long, c_uint, c_uint32, c_ulong, c_void_p

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
FAKE_DIR = os.path.join(ROOT, "tests", "fakehip")
# SLLM_FAKEHIP_SAN=1: the ASan + UBSan build of the same sources (tests/test_sanitizers.py)
FAKE_NAME = "libsllm_gfx950_fakehip_san.so" if os.environ.get("SLLM_FAKEHIP_SAN") else "libsllm_gfx950_fakehip.so"
FAKE = os.path.join(FAKE_DIR, FAKE_NAME)

HIP_INVALID_VALUE, HIP_OUT_OF_MEMORY = 1, 2          # hipErrorInvalidValue, hipErrorOutOfMemory
NOMEM, UNSUPPORTED, NO_DEVICE, HIP = -2, -4, -60, -61

TINY = dict(n_layer=2, n_embd=256, n_ff=512, n_head=4, n_head_kv=2, n_rot=64, n_vocab=300,
            eps=1e-5, rope_base=10000.0)


def _build():
    import fcntl
    # one build at a time when test workers run side by side
    with open(os.path.join(FAKE_DIR, ".build.lock"), "w") as lock:
        fcntl.flock(lock, fcntl.LOCK_EX)
        r = subprocess.run(["make", "-s", "-C", FAKE_DIR, FAKE_NAME], capture_output=True, text=True)
    if r.returncode != 0:
        pytest.fail(f"building the fake-HIP library failed:\n{r.stdout}\n{r.stderr}")


@pytest.fixture(scope="module")
def fake(amd):
    _build()
    L = amd._bind(FAKE, amd.PROTOTYPES)
    for name, res, args in (("fakehip_fail", None, [c_char_p, c_int, c_uint]), ("fakehip_clear", None, []),
                            ("fakehip_fired", c_int, []), ("fakehip_live", c_long, []),
                            ("fakehip_calls", c_ulong, [])):
        f = getattr(L, name)
        f.restype, f.argtypes = res, args
    yield L
    L.sllm_gfx950_close()


def _err(L):
    return L.sllm_gfx950_last_error().decode(errors="replace")


class Env:
    """Objects the scenarios use, created with nothing failing."""

    def __init__(self, amd, L):
        self.amd, self.L = amd, L
        self.keep = []
        self.n_rows, self.n = 256, 2560
        w = amd.synth_i2s(amd.synth_seed(9, 0, 0, 0), self.n_rows, self.n)
        self.w_host = w
        self.w = self.put(w)
        x = amd.synth_normal(3, 4 * self.n)
        self.x = self.put(x)
        self.q = self.alloc(4 * self.n)
        self.act = self.alloc(64)
        self.out = self.alloc(4 * 4 * self.n_rows)
        self.out_i = self.alloc(4 * 4 * self.n_rows)
        self.scratch = self.alloc(1 << 16)
        self.partials = self.alloc(4 * 16)
        self.jobs = (amd.GemvJob * 2)(
            amd.GemvJob(self.w, self.n_rows, self.n, self.x, None, None, self.out, None),
            amd.GemvJob(self.w, self.n_rows, self.n, self.x, None, None, None, self.out_i))
        self.plan = c_void_p()
        assert L.sllm_gfx950_plan_create(self.jobs, 2, byref(self.plan)) == 0
        self.gemm_jobs = (amd.GemmJob * 2)(amd.GemmJob(self.w, self.n_rows, self.out, None),
                                           amd.GemmJob(self.w, self.n_rows, None, self.out_i))
        gp = (amd.GemmPlanJob * 1)(amd.GemmPlanJob(self.w, self.n_rows, self.n, self.q, self.act, self.out, None))
        self.gemm_plan = c_void_p()
        assert L.sllm_gfx950_gemm_plan_create(gp, 1, 4, byref(self.gemm_plan)) == 0, _err(L)
        assert L.sllm_gfx950_events_reserve(4) == 0
        assert L.sllm_gfx950_event_record(0) == 0 and L.sllm_gfx950_event_record(1) == 0
        # a tiny model, as host arrays and as a GGUF image
        from oracle.gguf_synth import gguf_image
        self.model = amd.synth_model(TINY, 5)
        self.desc, self.desc_keep = amd.model_desc(self.model)
        self.image = np.frombuffer(gguf_image(self.model), np.uint8)
        self.m = c_void_p()
        assert L.sllm_gfx950_model_upload(byref(self.desc), byref(self.m)) == 0, _err(L)
        self.c = c_void_p()
        assert L.sllm_gfx950_ctx_new(self.m, 64, byref(self.c)) == 0, _err(L)
        self.logits = np.zeros(8 * TINY["n_vocab"], np.float32)
        self.tokens = np.array([1, 2, 3, 4, 5, 6], np.int32)
        self.ids = np.zeros(16, np.int32)
        hd = TINY["n_embd"] // TINY["n_head"]
        self.kv = np.zeros(TINY["n_layer"] * TINY["n_head_kv"] * 8 * hd, np.float32)
        self.t_dots = self.alloc(4 * L.sllm_gfx950_trace_dots(self.m))
        self.t_acts = self.alloc(8 * (4 * TINY["n_layer"] + 8))
        # the context's buffers made on first use (chunk staging, ...) exist
        # before any call is made to fail: a failure then has nothing to keep
        P_ = lambda a: a.ctypes.data_as(c_void_p)
        assert L.sllm_gfx950_forward_chunk(self.m, self.c, P_(self.tokens), 5, 0, P_(self.logits)) == 0, _err(L)
        self.reset_ctx(0)
        assert L.sllm_gfx950_generate_greedy(self.m, self.c, P_(self.tokens), 3, 2, P_(self.ids)) == 0, _err(L)
        self.reset_ctx(0)

    def alloc(self, n):
        p = c_void_p()
        assert self.L.sllm_gfx950_malloc(byref(p), n) == 0
        self.keep.append(p)
        return p.value

    def put(self, a):
        p = self.alloc(a.nbytes)
        assert self.L.sllm_gfx950_h2d(c_void_p(p), a.ctypes.data_as(c_void_p), a.nbytes) == 0
        return p

    def reset_ctx(self, n_past=0):
        L = self.L
        assert L.sllm_gfx950_ctx_reset(self.c) == 0
        for pos in range(n_past):
            assert L.sllm_gfx950_forward(self.m, self.c, int(self.tokens[pos]), pos, None) == 0, _err(L)

    def close(self):
        L = self.L
        if self.keep:
            L.sllm_gfx950_ctx_free(self.c)
            L.sllm_gfx950_model_free(self.m)
            L.sllm_gfx950_plan_destroy(self.plan)
            L.sllm_gfx950_gemm_plan_destroy(self.gemm_plan)
            for p in self.keep:
                L.sllm_gfx950_free(p)
        self.keep = []


def P(a):
    return a.ctypes.data_as(c_void_p)


_EVENTS = [8]


def scenarios(E):
    """(name, prepare, call -> (status, object), cleanup(object)) for every
    status-returning entry point that reaches the device."""
    L, amd = E.L, E.amd
    V = c_void_p
    nr, n = E.n_rows, E.n
    nothing = lambda: None
    ms = c_float()
    out = []

    def add(name, call, prepare=nothing, cleanup=None, freed=0, settle=nothing):
        out.append((name, prepare, call, cleanup, freed, settle))

    def st(v):
        return v, None

    def malloc():
        p = c_void_p()
        return L.sllm_gfx950_malloc(byref(p), 4096), p

    add("malloc", malloc, cleanup=lambda p: L.sllm_gfx950_free(p))
    host = np.zeros(64, np.uint8)
    add("h2d", lambda: st(L.sllm_gfx950_h2d(V(E.scratch), P(host), 64)))
    add("d2h", lambda: st(L.sllm_gfx950_d2h(P(host), V(E.scratch), 64)))
    add("sync", lambda: st(L.sllm_gfx950_sync()))
    add("timer", lambda: st(L.sllm_gfx950_timer_start() or L.sllm_gfx950_timer_stop(byref(ms))))
    _EVENTS[0] += 8                     # more events than before, so that it creates some
    target = _EVENTS[0]

    def events_reserve():
        return L.sllm_gfx950_events_reserve(target), None

    add("events_reserve", events_reserve)
    add("event_record", lambda: st(L.sllm_gfx950_event_record(2)))
    add("event_elapsed", lambda: st(L.sllm_gfx950_event_elapsed(0, 1, byref(ms))))
    add("copy", lambda: st(L.sllm_gfx950_copy(V(E.scratch), V(E.x), 4096)))
    add("checksum", lambda: st(L.sllm_gfx950_checksum(V(E.x), 4096, V(E.partials), 16)))
    add("diag_expf", lambda: st(L.sllm_gfx950_diag_expf(0, 1, 256, V(E.scratch))))
    add("quant_act", lambda: st(L.sllm_gfx950_quant_act(V(E.x), n, 2, V(E.q), V(E.act))))
    add("gemv", lambda: st(L.sllm_gfx950_gemv(V(E.w), nr, n, V(E.q), V(E.out_i))))
    add("gemv_epilogue", lambda: st(L.sllm_gfx950_gemv_epilogue(V(E.w), nr, n, V(E.q), V(E.act), V(E.out))))
    add("linear", lambda: st(L.sllm_gfx950_linear(V(E.w), nr, n, V(E.x), V(E.q), V(E.act), V(E.out))))
    add("linear_scratch", lambda: st(L.sllm_gfx950_linear(V(E.w), nr, n, V(E.x), None, None, V(E.out))))
    add("gemv_batch", lambda: st(L.sllm_gfx950_gemv_batch(E.jobs, 2)))
    add("gemv_batch_noalloc", lambda: st(L.sllm_gfx950_gemv_batch_noalloc(E.jobs, 2)))

    def plan_create():
        p = c_void_p()
        return L.sllm_gfx950_plan_create(E.jobs, 2, byref(p)), p

    add("plan_create", plan_create, cleanup=lambda p: L.sllm_gfx950_plan_destroy(p))
    add("plan_run", lambda: st(L.sllm_gfx950_plan_run(E.plan)))
    add("plan_run_marked", lambda: st(L.sllm_gfx950_plan_run_marked(E.plan, 3)))
    add("gemm", lambda: st(L.sllm_gfx950_gemm(V(E.w), nr, n, V(E.q), V(E.act), 4, V(E.out), None)))
    add("gemm_multi", lambda: st(L.sllm_gfx950_gemm_multi(ctypes.cast(E.gemm_jobs, V), 2, n, V(E.q),
                                                           V(E.act), 4)))
    add("linear_batch", lambda: st(L.sllm_gfx950_linear_batch(V(E.w), nr, n, V(E.x), 4, V(E.q), V(E.act),
                                                               V(E.out), None)))
    gp_jobs = (amd.GemmPlanJob * 2)(amd.GemmPlanJob(E.w, nr, n, E.q, E.act, E.out, None),
                                    amd.GemmPlanJob(E.w, nr, n, E.q, E.act, None, E.out_i))

    def gemm_plan_create():
        p = c_void_p()
        return L.sllm_gfx950_gemm_plan_create(gp_jobs, 2, 4, byref(p)), p

    add("gemm_plan_create", gemm_plan_create, cleanup=lambda p: L.sllm_gfx950_gemm_plan_destroy(p))
    add("gemm_plan_run", lambda: st(L.sllm_gfx950_gemm_plan_run(E.gemm_plan)))

    def register():
        return L.sllm_gfx950_tensor_register(P(E.w_host), nr, n), None

    add("tensor_register", register, cleanup=lambda _: L.sllm_gfx950_tensor_unregister(P(E.w_host)))
    # the device copy goes even when the wait before freeing it fails
    add("tensor_unregister", lambda: st(L.sllm_gfx950_tensor_unregister(P(E.w_host))),
        prepare=lambda: L.sllm_gfx950_tensor_register(P(E.w_host), nr, n), freed=1)
    # the kernel row's upload on first use, and the release hook
    add("tensor_acquire", lambda: st(L.sllm_gfx950_tensor_acquire(P(E.w_host), nr, n)),
        cleanup=lambda _: L.sllm_gfx950_tensor_release_acquired())
    add("tensor_release_acquired", lambda: st(L.sllm_gfx950_tensor_release_acquired()),
        prepare=lambda: L.sllm_gfx950_tensor_acquire(P(E.w_host), nr, n), freed=1)

    # decode
    def upload():
        m = c_void_p()
        return L.sllm_gfx950_model_upload(byref(E.desc), byref(m)), m

    add("model_upload", upload, cleanup=lambda m: L.sllm_gfx950_model_free(m))

    def load_gguf():
        m = c_void_p()
        return L.sllm_gfx950_model_load_gguf(P(E.image), E.image.nbytes, byref(m)), m

    add("model_load_gguf", load_gguf, cleanup=lambda m: L.sllm_gfx950_model_free(m))

    def ctx_new():
        c = c_void_p()
        return L.sllm_gfx950_ctx_new(E.m, 32, byref(c)), c

    add("ctx_new", ctx_new, cleanup=lambda c: L.sllm_gfx950_ctx_free(c))
    add("ctx_reset", lambda: st(L.sllm_gfx950_ctx_reset(E.c)), prepare=lambda: E.reset_ctx(2))
    add("forward", lambda: st(L.sllm_gfx950_forward(E.m, E.c, 7, 2, P(E.logits))), prepare=lambda: E.reset_ctx(2))
    add("forward_no_logits", lambda: st(L.sllm_gfx950_forward(E.m, E.c, 7, 2, None)),
        prepare=lambda: E.reset_ctx(2))

    def graph_on():
        assert L.sllm_gfx950_ctx_set_graph(E.c, 0) == 0
        E.reset_ctx(2)
        assert L.sllm_gfx950_ctx_set_graph(E.c, 1) == 0

    # a graph captured before the failure stays with the context for replay;
    # switching graphs off releases it
    add("forward_graph", lambda: st(L.sllm_gfx950_forward(E.m, E.c, 7, 2, P(E.logits))), prepare=graph_on,
        cleanup=lambda _: L.sllm_gfx950_ctx_set_graph(E.c, 0),
        settle=lambda: L.sllm_gfx950_ctx_set_graph(E.c, 0))
    add("forward_chunk", lambda: st(L.sllm_gfx950_forward_chunk(E.m, E.c, P(E.tokens), 5, 1, P(E.logits))),
        prepare=lambda: E.reset_ctx(1))
    add("forward_chunk_last", lambda: st(L.sllm_gfx950_forward_chunk(E.m, E.c, P(E.tokens), 5, 1, None)),
        prepare=lambda: E.reset_ctx(1))
    add("prefill_chunked", lambda: st(L.sllm_gfx950_forward_prefill_chunked(E.m, E.c, P(E.tokens), 6, 4,
                                                                              P(E.logits))),
        prepare=lambda: E.reset_ctx(0))

    def greedy_prep():
        E.reset_ctx(0)
        assert L.sllm_gfx950_ctx_set_inflight(E.c, 2) == 0

    add("generate_greedy", lambda: st(L.sllm_gfx950_generate_greedy(E.m, E.c, P(E.tokens), 3, 5, P(E.ids))),
        prepare=greedy_prep)
    tok = c_int32()
    add("ctx_argmax", lambda: st(L.sllm_gfx950_ctx_argmax(E.c, byref(tok))), prepare=lambda: E.reset_ctx(1))
    add("ctx_kv_load", lambda: st(L.sllm_gfx950_ctx_kv_load(E.c, P(E.kv), P(E.kv), 8, P(E.logits))),
        prepare=lambda: E.reset_ctx(0))

    def trace_prep():
        E.reset_ctx(0)

    def trace():
        s = L.sllm_gfx950_ctx_trace(E.c, V(E.t_dots), V(E.t_acts))
        if s == 0:
            s = L.sllm_gfx950_forward(E.m, E.c, 7, 0, P(E.logits))
        return s, None

    add("ctx_trace", trace, prepare=trace_prep)
    return out


def _sweep(L, name, prepare, call, cleanup, freed, settle, fn, err, want):
    """Fail the k-th matching HIP call for k = 0, 1, ... until the call
    completes without reaching a k-th one. Returns the number of failure
    points. `freed`: HIP objects the call releases even when it fails."""
    k = 0
    while True:
        prepare()
        live = L.fakehip_live()
        L.fakehip_fail(fn.encode(), err, k)
        status, obj = call()
        fired = L.fakehip_fired()
        L.fakehip_clear()
        if not fired:
            assert status == 0, f"{name}: status {status} with nothing failing: {_err(L)}"
            if cleanup is not None:
                cleanup(obj)
            return k
        assert status == want, f"{name}: failing {fn} #{k} gave {status}, not {want}: {_err(L)}"
        assert _err(L), name
        settle()
        assert L.fakehip_live() == live - freed, \
            f"{name}: failing {fn} #{k} left {L.fakehip_live() - live + freed} HIP objects"
        k += 1
        assert k < 5000, f"{name}: no end to the HIP calls"


@pytest.fixture(scope="module")
def env(amd, fake):
    assert fake.sllm_gfx950_open(0) == 0, _err(fake)
    E = Env(amd, fake)
    yield E
    E.close()


def test_every_failed_allocation_returns_nomem(env):
    """Out of device or pinned memory at every allocation of every entry
    point: -2, nothing left allocated."""
    points = {}
    for name, *s in scenarios(env):
        points[name] = (_sweep(env.L, name, *s, "hipMalloc", HIP_OUT_OF_MEMORY, NOMEM) +
                        _sweep(env.L, name, *s, "hipHostMalloc", HIP_OUT_OF_MEMORY, NOMEM))
    # the calls that allocate were driven through their allocations
    for name in ("malloc", "plan_create", "gemv_batch", "tensor_register", "tensor_acquire", "model_upload",
                 "model_load_gguf", "ctx_new", "gemm_plan_create"):
        assert points[name] > 0, name


def test_every_failed_hip_call_returns_hip_error(env):
    """Any other HIP failure at every HIP call of every entry point: -61,
    nothing left allocated, and the call then succeeds."""
    for name, *s in scenarios(env):
        assert _sweep(env.L, name, *s, "*", HIP_INVALID_VALUE, HIP) > 0, name


def test_streamed_plan_tables_for_many_uneven_tensors(amd, env):
    """A plan of at most four tokens streams (i2s_kernels.hip: gemm_stream_body):
    the host cuts its 128-row tiles into runs of about equal iterations, at
    most 64 tiles a run. 20,000 one-iteration tiles beside 200 tiles of 128
    iterations make runs that want more than 64 tiles, so the cut is redone
    with more runs until every run fits; the tables must come out whole (the
    sanitizer build runs this too) and the plan must run and free cleanly."""
    L = env.L
    w_small = env.put(amd.synth_i2s(amd.synth_seed(9, 1, 64, 256), 64, 256))
    w_big = env.put(amd.synth_i2s(amd.synth_seed(9, 2, 256, 65536), 256, 65536))
    q, act = env.alloc(4 * 65536), env.alloc(64)
    out_small, out_big = env.alloc(4 * 4 * 64), env.alloc(4 * 4 * 256)
    # the big tensors first: the runs after them, cut for about 108
    # iterations, stop at 64 one-iteration tiles (37 re-cuts, 717 runs)
    jobs = [amd.GemmPlanJob(w_big, 256, 65536, q, act, out_big, None) for _ in range(100)]
    jobs += [amd.GemmPlanJob(w_small, 64, 256, q, act, out_small, None) for _ in range(20000)]
    arr = (amd.GemmPlanJob * len(jobs))(*jobs)
    p = c_void_p()
    assert L.sllm_gfx950_gemm_plan_create(arr, len(jobs), 4, byref(p)) == 0, _err(L)
    try:
        assert L.sllm_gfx950_gemm_plan_run(p) == 0, _err(L)
    finally:
        L.sllm_gfx950_gemm_plan_destroy(p)


def test_open_failures_leave_the_library_closed(amd, fake, env):
    """A failed open -- at each of its HIP calls -- returns -61 (or -60 when
    the runtime reports no device), leaves nothing behind and the library
    closed; the next open works."""
    L = fake
    env.close()
    L.sllm_gfx950_close()
    assert L.fakehip_live() == 0
    k = 0
    while True:
        L.fakehip_fail(b"*", HIP_INVALID_VALUE, k)
        status = L.sllm_gfx950_open(0)
        fired = L.fakehip_fired()
        L.fakehip_clear()
        if not fired:
            assert status == 0
            break
        assert status == HIP, (k, status, _err(L))
        assert not L.sllm_gfx950_is_open()
        assert L.fakehip_live() == 0, f"open: failing HIP call #{k} left {L.fakehip_live()} objects"
        k += 1
    assert k >= 8        # device count, properties, set device, two modules, functions, stream, events, ...
    L.sllm_gfx950_close()
    L.fakehip_fail(b"hipModuleLoadData", HIP_INVALID_VALUE, 0)
    assert L.sllm_gfx950_open(0) == HIP and "hipModuleLoadData" in _err(L)
    L.fakehip_clear()
    L.fakehip_fail(b"hipGetDeviceCount", 100, 0)                # hipErrorNoDevice
    assert L.sllm_gfx950_open(0) == NO_DEVICE
    L.fakehip_clear()
    assert L.sllm_gfx950_open(0) == 0
    env.__init__(amd, L)            # the module's objects again, for any later test


def test_entry_points_before_open_report_no_device(amd):
    """-60 from every device and decode entry point while the library is not
    open (a separate process: this one's fake device is open)."""
    _build()
    code = f"""
import ctypes, sys
sys.path.insert(0, {ROOT!r})
sys.path.insert(0, {os.path.join(ROOT, "tests")!r})
from conftest import load_package
amd = load_package()
L = amd._bind({FAKE!r}, amd.PROTOTYPES)
V = ctypes.c_void_p
p = V(); ms = ctypes.c_float(); t = ctypes.c_int32()
import numpy as np
from oracle.gguf_synth import gguf_image
# a valid image: the loader checks the file first, as sllm_gguf_open does,
# and needs the device only to upload
image = np.frombuffer(gguf_image(amd.synth_model({TINY!r}, 1)), np.uint8)
calls = {{
  "malloc": lambda: L.sllm_gfx950_malloc(ctypes.byref(p), 64),
  "h2d": lambda: L.sllm_gfx950_h2d(None, None, 0), "d2h": lambda: L.sllm_gfx950_d2h(None, None, 0),
  "sync": lambda: L.sllm_gfx950_sync(), "timer_start": lambda: L.sllm_gfx950_timer_start(),
  "timer_stop": lambda: L.sllm_gfx950_timer_stop(ctypes.byref(ms)),
  "events_reserve": lambda: L.sllm_gfx950_events_reserve(2), "event_record": lambda: L.sllm_gfx950_event_record(0),
  "event_elapsed": lambda: L.sllm_gfx950_event_elapsed(0, 1, ctypes.byref(ms)),
  "copy": lambda: L.sllm_gfx950_copy(None, None, 16), "checksum": lambda: L.sllm_gfx950_checksum(None, 16, None, 1),
  "diag_expf": lambda: L.sllm_gfx950_diag_expf(0, 1, 1, None),
  "quant_act": lambda: L.sllm_gfx950_quant_act(None, 128, 1, None, None),
  "gemv": lambda: L.sllm_gfx950_gemv(None, 1, 128, None, None),
  "gemv_epilogue": lambda: L.sllm_gfx950_gemv_epilogue(None, 1, 128, None, None, None),
  "linear": lambda: L.sllm_gfx950_linear(None, 1, 128, None, None, None, None),
  "gemv_batch": lambda: L.sllm_gfx950_gemv_batch(None, 1),
  "gemv_batch_noalloc": lambda: L.sllm_gfx950_gemv_batch_noalloc(None, 1),
  "plan_create": lambda: L.sllm_gfx950_plan_create(None, 1, ctypes.byref(p)),
  "plan_run": lambda: L.sllm_gfx950_plan_run(None), "plan_run_marked": lambda: L.sllm_gfx950_plan_run_marked(None, 0),
  "gemm": lambda: L.sllm_gfx950_gemm(None, 1, 128, None, None, 1, None, None),
  "gemm_multi": lambda: L.sllm_gfx950_gemm_multi(None, 1, 128, None, None, 1),
  "linear_batch": lambda: L.sllm_gfx950_linear_batch(None, 1, 128, None, 1, None, None, None, None),
  "gemm_plan_create": lambda: L.sllm_gfx950_gemm_plan_create(None, 1, 1, ctypes.byref(p)),
  "gemm_plan_run": lambda: L.sllm_gfx950_gemm_plan_run(None),
  "tensor_register": lambda: L.sllm_gfx950_tensor_register(None, 1, 128),
  "tensor_unregister": lambda: L.sllm_gfx950_tensor_unregister(None),
  "tensor_acquire": lambda: L.sllm_gfx950_tensor_acquire(None, 1, 128),
  "tensor_release_acquired": lambda: L.sllm_gfx950_tensor_release_acquired(),
  "device_info": lambda: L.sllm_gfx950_device_info(None, 0, None, None),
  "model_upload": lambda: L.sllm_gfx950_model_upload(None, ctypes.byref(p)),
  "model_load_gguf": lambda: L.sllm_gfx950_model_load_gguf(image.ctypes.data_as(V), image.size, ctypes.byref(p)),
  "ctx_new": lambda: L.sllm_gfx950_ctx_new(None, 16, ctypes.byref(p)),
  "ctx_reset": lambda: L.sllm_gfx950_ctx_reset(None),
  "forward": lambda: L.sllm_gfx950_forward(None, None, 0, 0, None),
  "forward_chunk": lambda: L.sllm_gfx950_forward_chunk(None, None, None, 1, 0, None),
  "prefill_chunked": lambda: L.sllm_gfx950_forward_prefill_chunked(None, None, None, 1, 1, None),
  "generate_greedy": lambda: L.sllm_gfx950_generate_greedy(None, None, None, 0, 1, None),
  "ctx_argmax": lambda: L.sllm_gfx950_ctx_argmax(None, ctypes.byref(t)),
  "ctx_kv_load": lambda: L.sllm_gfx950_ctx_kv_load(None, None, None, 0, None),
  "ctx_set_inflight": lambda: L.sllm_gfx950_ctx_set_inflight(None, 1),
  "ctx_set_graph": lambda: L.sllm_gfx950_ctx_set_graph(None, 1),
  "ctx_trace": lambda: L.sllm_gfx950_ctx_trace(None, None, None),
}}
bad = {{k: f() for k, f in calls.items()}}
bad = {{k: v for k, v in bad.items() if v != {NO_DEVICE}}}
print("NOT-60", bad)
sys.exit(1 if bad else 0)
"""
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr


ROW_CALLS = {
    "quant_act": ("L.sllm_gfx950_i2s_quant_act(P(x), 256, P(q), ctypes.byref(a))",
                  "sllm_gfx950_i2s_quant_act failed"),
    "gemv": ("L.sllm_gfx950_i2s_gemv(P(w), 64, 256, P(q), P(o))", "sllm_gfx950_i2s_gemv failed"),
    "dot": ("L.sllm_gfx950_i2s_dot(P(w), P(q), 256)", "sllm_gfx950_i2s_gemv failed"),
    "kdispatch_gemv": ("L.sllm_kdispatch_select(b'gfx950'); L.sllm_kdispatch_gemv(P(w), 64, 256, P(q), P(o))",
                       "sllm_gfx950_i2s_gemv failed"),
}


def _row_child(call, fail, opened=True):
    return f"""
import ctypes, sys
import numpy as np
sys.path.insert(0, {os.path.join(ROOT, "tests")!r})
from conftest import load_package
amd = load_package()
L = amd._bind({FAKE!r}, amd.PROTOTYPES)
L.fakehip_fail.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.c_uint]
P = lambda a: a.ctypes.data_as(ctypes.c_void_p)
w = amd.synth_i2s(1, 64, 256); x = np.ones(256, np.float32); q = np.ones(256, np.int8)
o = np.zeros(64, np.int32); a = amd.Act()
if {opened!r}:
    assert L.sllm_gfx950_open(0) == 0
    assert L.sllm_gfx950_tensor_register(P(w), 64, 256) == 0
{"L.fakehip_fail(b'*', 1, 0)" if fail else "pass"}
{call}
print("returned", flush=True)
"""


@pytest.mark.parametrize("which", sorted(ROW_CALLS))
def test_host_pointer_row_aborts_with_its_message(which):
    """A HIP failure inside the host-pointer row: the reason on stderr, then
    abort -- no status to return, and zeros would read as a wrong answer."""
    _build()
    call, msg = ROW_CALLS[which]
    r = subprocess.run([sys.executable, "-c", _row_child(call, True)], capture_output=True, text=True, timeout=120)
    assert r.returncode == -6, (r.returncode, r.stdout, r.stderr)
    assert "returned" not in r.stdout
    assert msg in r.stderr and "hip-error" in r.stderr, r.stderr
    # and with nothing failing, the same call returns
    r = subprocess.run([sys.executable, "-c", _row_child(call, False)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and "returned" in r.stdout, r.stderr


def test_row_without_device_or_selection_aborts_with_its_message():
    _build()
    r = subprocess.run([sys.executable, "-c", _row_child(ROW_CALLS["gemv"][0], False, opened=False)],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == -6 and "library not open" in r.stderr, r.stderr
    r = subprocess.run([sys.executable, "-c", _row_child("L.sllm_kdispatch_gemv(P(w), 64, 256, P(q), P(o))",
                                                         False, opened=False)],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == -6 and "no kernel row installed" in r.stderr, r.stderr

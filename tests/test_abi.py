"""The C ABI, the dispatch table and the workload generator, on CPU.

No kernel runs here: these tests check that libsllm_gfx950.so loads and
exports every function include/saphira_amd/*.h declares, that the product
fails loudly without a gfx950 device (no silent CPU fallback), the dispatch
table's selection rules, and the synthetic generator's layout.
"""
import ctypes
import glob
import os
import re
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_functions():
    names = set()
    for path in glob.glob(os.path.join(ROOT, "include", "saphira_amd", "*.h")):
        text = re.sub(r"/\*.*?\*/", "", open(path).read(), flags=re.S)
        text = re.sub(r"//[^\n]*", "", text)
        for m in re.finditer(r"\b(sllm_\w+)\s*\(", text):
            names.add(m.group(1))
    return names


def test_headers_declare_the_expected_surface():
    names = _declared_functions()
    for must in ("sllm_gfx950_open", "sllm_gfx950_quant_act", "sllm_gfx950_gemv",
                 "sllm_gfx950_gemv_epilogue", "sllm_gfx950_i2s_gemv", "sllm_gfx950_i2s_quant_act",
                 "sllm_gfx950_i2s_dot", "sllm_kdispatch_select", "sllm_kdispatch_gemv"):
        assert must in names


def test_library_exports_every_declared_function(amd):
    lib = amd.lib()
    names = _declared_functions()
    missing = [n for n in sorted(names) if not hasattr(lib, n)]
    assert not missing, missing
    # and the bindings describe each of them
    assert names <= set(amd.PROTOTYPES), sorted(names - set(amd.PROTOTYPES))


def test_library_embeds_a_gfx950_code_object():
    out = subprocess.run(["nm", "-D", "--defined-only", os.path.join(ROOT, "saphira-llm_amd", "libsllm_gfx950.so")],
                         capture_output=True, text=True, check=True).stdout
    assert "sllm_gfx950_open" in out
    blob = open(os.path.join(ROOT, "saphira-llm_amd", "libsllm_gfx950.so"), "rb").read()
    assert b"amdgcn-amd-amdhsa--gfx950" in blob
    for k in (b"sllm_k_quant_act", b"sllm_k_quant_list", b"sllm_k_gemv_slab", b"sllm_k_gemv_stream_l4",
              b"sllm_k_gemv_stream_l8", b"sllm_k_gemv_stream_l16", b"sllm_k_gemm_mfma_s1x1",
              b"sllm_k_gemm_mfma_2x2", b"sllm_k_gemm_mfma_4x2", b"sllm_k_gemm_mfma_l128",
              b"sllm_k_gemm_mfma_l128s", b"sllm_k_gemm_dl1x1", b"sllm_k_gemm_dl2x1", b"sllm_k_gemm_dl2x2",
              b"sllm_k_gemm_dl4x4"):
        assert k in blob


def _has_gpu(amd):
    return amd.lib().sllm_gfx950_open(0) == 0


def test_open_without_a_gfx950_reports_no_device(amd):
    lib = amd.lib()
    st = lib.sllm_gfx950_open(0)
    if st == 0:
        pytest.skip("a gfx950 is present; covered by the gpu tests")
    assert st == -60, (st, lib.sllm_gfx950_last_error())
    assert lib.sllm_gfx950_is_open() == 0
    p = ctypes.c_void_p()
    assert lib.sllm_gfx950_malloc(ctypes.byref(p), 16) == -60
    assert lib.sllm_gfx950_gemv(None, 1, 128, None, None) in (-60, -1)
    assert lib.sllm_gfx950_status_string(-60) == b"no-gfx950-device"


_ABORT_SNIPPET = r"""
import sys, ctypes, importlib.util, numpy as np
spec = importlib.util.spec_from_file_location("saphira_llm_amd", sys.argv[1])
m = importlib.util.module_from_spec(spec); spec.loader.exec_module(m)
lib = m.lib()
w = np.zeros(128 // 4 * 2 + 32, np.uint8); q = np.zeros(128, np.int8); out = np.zeros(2, np.int32)
getattr(lib, sys.argv[2])(*{
  "sllm_gfx950_i2s_gemv": (m.ptr(w), 2, 128, m.ptr(q), m.ptr(out)),
  "sllm_kdispatch_gemv": (m.ptr(w), 2, 128, m.ptr(q), m.ptr(out)),
}[sys.argv[2]])
print("returned", out)
"""


@pytest.mark.parametrize("fn", ["sllm_gfx950_i2s_gemv", "sllm_kdispatch_gemv"])
def test_hot_path_without_a_device_aborts_loudly(amd, fn):
    """The reference's void kernel signatures cannot return a status; with no
    device open (or no row installed) they must stop, not compute on the CPU."""
    if _has_gpu(amd):
        pytest.skip("a gfx950 is present")
    r = subprocess.run([sys.executable, "-c", _ABORT_SNIPPET, os.path.join(ROOT, "saphira-llm_amd", "__init__.py"), fn],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode != 0 and "returned" not in r.stdout
    assert "no kernel row installed" in r.stderr or "library not open" in r.stderr, r.stderr


def test_dispatch_table_rules(amd):
    lib = amd.lib()
    if _has_gpu(amd):
        pytest.skip("selection without a device is the case under test")
    assert lib.sllm_kdispatch_count() >= 1
    assert lib.sllm_kdispatch_row(0).contents.name == b"gfx950"
    lib.sllm_kdispatch_reset()
    assert not lib.sllm_kdispatch_installed()
    assert lib.sllm_kdispatch_installed_name() == b"none"
    # the gfx950 row cannot open here: selection fails, nothing is installed
    assert lib.sllm_kdispatch_select(b"gfx950") == -60
    assert not lib.sllm_kdispatch_installed()
    assert lib.sllm_kdispatch_select(b"no-such-row") == -1

    # a host row registered by the integrator (a counting stub, not a kernel)
    calls = []
    row = amd.KernelRow()
    row.name = b"test-stub"
    row.priority = 1
    row.open = row._fields_[2][1](lambda: 0)
    row.quant_act = row._fields_[3][1](lambda x, n, q, a: calls.append(("quant", n)))
    row.dot = row._fields_[4][1](lambda w, q, n: calls.append(("dot", n)) or 7)
    row.gemv = row._fields_[5][1](lambda w, r, n, q, o: calls.append(("gemv", r, n)))
    row.release = row._fields_[6][1](lambda: calls.append(("release",)))
    test_dispatch_table_rules._keep = row      # callbacks must outlive the table
    if lib.sllm_kdispatch_count() == 1:
        assert lib.sllm_kdispatch_register(ctypes.byref(row)) == 0
    assert lib.sllm_kdispatch_register(ctypes.byref(row)) == -1          # duplicate name
    # "auto" tries gfx950 (priority 100) first, then the stub
    assert lib.sllm_kdispatch_select(b"auto") == 0
    assert lib.sllm_kdispatch_installed().contents.name == b"test-stub"
    assert lib.sllm_kdispatch_installed_name() == b"test-stub"
    assert lib.sllm_kdispatch_dot(None, None, 256) == 7
    lib.sllm_kdispatch_gemv(None, 3, 384, None, None)
    lib.sllm_kdispatch_release()
    assert calls[-3:] == [("dot", 256), ("gemv", 3, 384), ("release",)]
    lib.sllm_kdispatch_reset()
    lib.sllm_kdispatch_release()                   # nothing installed: nothing happens
    assert calls[-1] == ("release",) and len([c for c in calls if c == ("release",)]) == 1


# ---------------------------------------------------------------------------
# synthetic workloads
# ---------------------------------------------------------------------------

def test_synth_packs_in_the_converter_layout(amd, orc):
    seed = amd.synth_seed(1, 2, 3, 4)
    n_rows, n = 5, 640
    packed = amd.synth_i2s(seed, n_rows, n, threads=1)
    codes = amd.synth_codes(seed, n_rows, n)
    want = np.concatenate([orc.pack_converter(r)[: n // 4] for r in codes])
    np.testing.assert_array_equal(packed[: n_rows * n // 4], want)
    assert orc.scale(packed, n_rows * n) == amd.synth_scale(seed)
    assert not packed[n_rows * n // 4 + 4:].any()


def test_synth_is_deterministic_and_thread_count_invariant(amd):
    seed = amd.synth_seed(1, 0, 0, 1)
    a = amd.synth_i2s(seed, 300, 2560, threads=1)
    b = amd.synth_i2s(seed, 300, 2560, threads=7)
    np.testing.assert_array_equal(a, b)
    c = amd.synth_i2s(seed + 1, 300, 2560, threads=7)
    assert (a != c).any()


def test_synth_distributions(amd):
    codes = amd.synth_codes(amd.synth_seed(0, 1), 64, 4096)
    frac = np.bincount(codes.ravel(), minlength=3) / codes.size
    assert codes.max() <= 2 and np.all(np.abs(frac - 1 / 3) < 0.01)
    scales = [amd.synth_scale(amd.synth_seed(0, s)) for s in range(200)]
    assert min(scales) >= 0.5 and max(scales) < 2.0
    x = amd.synth_normal(123, 200001)
    assert abs(float(x.mean())) < 0.01 and abs(float(x.std()) - 1) < 0.01
    assert x.dtype == np.float32 and np.isfinite(x).all()

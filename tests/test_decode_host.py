"""The decode step's host side, on CPU: the C library's expf restated for
the GPU (every one of the 2^32 inputs), the decode entry points' presence
and their refusal without a device. The GPU runs are tests/test_gpu_decode.py.
"""
import ctypes
import os

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_expf_restatement_matches_the_c_library_on_every_input(amd):
    """csrc/libm_expf.h (the softmax's scalar tail on the GPU) against the
    host expf, all 2^32 bit patterns."""
    first = ctypes.c_uint32()
    bad = amd.synth_lib().sllm_expf_mismatches(0, 1 << 32, min(8, os.cpu_count() or 1), ctypes.byref(first))
    assert bad == 0, f"{bad} inputs differ, first 0x{first.value:08x}"


def test_decode_kernels_are_in_the_library():
    blob = open(os.path.join(ROOT, "saphira-llm_amd", "libsllm_gfx950.so"), "rb").read()
    for k in (b"sllm_k_dec_gemv", b"sllm_k_dec_scores", b"sllm_k_dec_pv", b"sllm_k_dec_lm_head"):
        assert k in blob


def test_decode_refuses_without_a_device(amd):
    lib = amd.lib()
    if lib.sllm_gfx950_open(0) == 0:
        pytest.skip("a gfx950 is present; covered by the gpu tests")
    model = amd.synth_model(dict(n_layer=1, n_embd=128, n_ff=128, n_head=2, n_head_kv=1, n_rot=64,
                                 n_vocab=16, eps=1e-5, rope_base=10000.0), 0)
    d, keep = amd.model_desc(model)
    m = ctypes.c_void_p()
    assert lib.sllm_gfx950_model_upload(ctypes.byref(d), ctypes.byref(m)) == -60
    assert not m.value
    c = ctypes.c_void_p()
    assert lib.sllm_gfx950_ctx_new(None, 8, ctypes.byref(c)) == -60


def test_trace_size_counts_every_projection(amd):
    # per block q (e) + k, v (gqa each) + o (e) + gate, up (f each) + down (e)
    from oracle import oracle as orc
    cfg = dict(amd.BITNET_2B)
    e, f = cfg["n_embd"], cfg["n_ff"]
    gqa = e // cfg["n_head"] * cfg["n_head_kv"]
    assert orc.n_trace_dots(cfg) == cfg["n_layer"] * (3 * e + 2 * gqa + 2 * f)

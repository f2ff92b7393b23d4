"""The integration patch (oracle/gfx950_forward.patch) on the CPU.

The patch is what a maintainer applies to the reference's src/forward.c to
install the gfx950 row (the GPU tests run the result against the unpatched
reference). Here: it only inserts lines, every insertion sits in an
SLLM_WITH_GFX950 conditional (so without the flag the reference compiles to
what it was), and a build with the flag refuses to load a model when no
gfx950 device is present (status SLLM_ERR_UNSUPPORTED, -4, from
include/saphira_llm/status.h:33) instead of falling back to its CPU kernels.
"""
import ctypes
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PATCH = os.path.join(ROOT, "oracle", "gfx950_forward.patch")


def _hunks():
    text = open(PATCH).read().splitlines()
    assert text[0].startswith("--- ") and text[1].startswith("+++ ")
    hunks, cur = [], None
    for line in text[2:]:
        if line.startswith("@@"):
            # a count of 1 is left out of a hunk header
            m = re.match(r"@@ -(\d+)(?:,(\d+))? \+(\d+)(?:,(\d+))? @@", line)
            assert m, line
            cur = (int(m.group(2) or 1), [])
            hunks.append(cur)
        else:
            assert line.startswith("+"), f"patch line is not an insertion: {line!r}"
            cur[1].append(line[1:])
    return hunks


def test_patch_only_inserts_conditional_lines():
    hunks = _hunks()
    assert all(removed == 0 for removed, _ in hunks)
    depth, seen_else = 0, 0
    for _, lines in hunks:
        for ln in lines:
            s = ln.strip()
            if s.startswith("#if"):
                assert s == "#ifdef SLLM_WITH_GFX950", s
                depth += 1
            elif s == "#else":
                seen_else += 1
            elif s == "#endif":
                depth -= 1
    assert depth == 0
    # the four quantiser sites and sllm_model_free keep the reference's line
    # as the #else branch
    assert seen_else == 5
    # outside the conditionals no code is inserted
    inside = 0
    for _, lines in hunks:
        for ln in lines:
            s = ln.strip()
            if s.startswith("#ifdef"):
                inside += 1
            elif s == "#endif":
                inside -= 1
            elif s and s != "#else" and inside == 0:
                assert False, f"inserted outside SLLM_WITH_GFX950: {ln!r}"


def test_patch_touches_the_documented_sites():
    """Row selection at load, the GEMV, four quantiser calls and the release
    hook in sllm_model_free: nothing in the loader (the row uploads each
    matrix on its first GEMV)."""
    body = "\n".join("\n".join(lines) for _, lines in _hunks())
    assert body.count('sllm_kdispatch_select("gfx950")') == 1
    assert body.count("sllm_kdispatch_gemv(") == 1
    assert body.count("sllm_kdispatch_quant_act(") == 4
    assert body.count("sllm_kdispatch_release();") == 1
    assert "sllm_gfx950_tensor_register" not in body and "gfx950_release" not in body
    # eight sites: the include / layout check, the GEMV, the select, sllm_model_free
    # (two hunks) and the four quantisers (two hunks each)
    assert len(_hunks()) == 13


def test_patched_reference_refuses_without_a_device(amd, orc):
    if not orc.ref_gfx950_available():
        pytest.skip("oracle/_ref was built without the reference tree")
    if amd.lib().sllm_gfx950_open(0) == 0:
        amd.lib().sllm_gfx950_close()
        pytest.skip("a gfx950 device is present: the GPU tests run the patched forward")
    from oracle.gguf_synth import gguf_image
    tiny = dict(n_layer=1, n_embd=128, n_ff=256, n_head=2, n_head_kv=1, n_rot=64, n_vocab=64,
                eps=1e-5, rope_base=10000.0)
    image = np.frombuffer(gguf_image(amd.synth_model(tiny, 1)), np.uint8)
    st = ctypes.c_int()
    lib = orc.ref_gfx950()
    assert not lib.ref_model_open(orc._p(image), image.nbytes, ctypes.byref(st))
    assert st.value == -4
    # the unpatched build loads the same image
    r = orc.ref().ref_model_open(orc._p(image), image.nbytes, ctypes.byref(st))
    assert r and st.value == 0
    orc.ref().ref_model_close(r)

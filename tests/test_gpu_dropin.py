"""The reference's own forward pass with the gfx950 row installed.

oracle/gfx950_forward.patch is the integration a maintainer applies to the
reference's src/forward.c: select the row at model load (after :334), send
sllm_gemv (:196-205) and the four quantiser calls (:651, :737, :763, :788)
through sllm_kdispatch_*, and let sllm_model_free (:457) call the row's
release hook. The row uploads each matrix on its first GEMV. The oracle recipe applies it to a copy of
forward.c and builds oracle/_ref/libsllm_ref_gfx950.so beside the unpatched
oracle/_ref/libsllm_ref.so. Both run the reference's own sllm_forward; one
reaches its CPU kernels, the other the GPU row. The row returns the CPU
kernels' int32 dots and activation scale / sum bit for bit and the reference's
own epilogue runs on them, so every logit must be bit-identical -- token by
token and through the chunk path (n > 1 tokens per sllm_gemv round).
"""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TINY = dict(n_layer=2, n_embd=256, n_ff=512, n_head=4, n_head_kv=2, n_rot=64, n_vocab=1000,
            eps=1e-5, rope_base=500000.0)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _tokens(n, vocab, seed):
    return [int(t) for t in np.random.default_rng(seed).integers(0, vocab, n)]


@pytest.fixture(scope="module")
def patched(amd, orc, dev):
    if not (orc.ref_available() and orc.ref_gfx950_available()):
        pytest.skip("oracle/_ref was built without the reference tree (make -C oracle ref)")
    lib = orc.ref_gfx950()
    yield lib
    amd.lib().sllm_kdispatch_reset()


def _pair(orc, lib, model, n_ctx):
    return orc.RefDecoder(model, n_ctx), orc.RefDecoder(model, n_ctx, lib=lib)


def _weights(amd, image):
    """Host addresses of every I2_S tensor inside a GGUF image."""
    st, cfg, tensors = amd.gguf_describe(image.tobytes())
    assert st == 0
    base = image.ctypes.data
    return [base + off for key, off in tensors.items()
            if isinstance(key, tuple) and key[1] in amd.LAYER_I2S]


def test_patched_forward_matches_reference_tiny(amd, orc, patched):
    model = amd.synth_model(TINY, 41)
    toks = _tokens(24, TINY["n_vocab"], 42)
    cpu, gpu = _pair(orc, patched, model, 48)
    try:
        print("[dropin] tiny: 24 tokens one at a time", flush=True)
        # the model load installed the device row (tests/test_i2s.c:500-537 asks the same of
        # the CPU rows through sllm_i2s_dot_isa)
        assert amd.lib().sllm_kdispatch_installed_name() == b"gfx950"
        for pos, t in enumerate(toks):
            a, b = cpu.forward(t, pos), gpu.forward(t, pos)
            assert np.array_equal(bits(a), bits(b)), pos
            assert orc.ref().ref_argmax(orc._p(a), a.size) == patched.ref_argmax(orc._p(b), b.size)
        print("[dropin] tiny: a 9-token chunk at position 24", flush=True)
        more = _tokens(9, TINY["n_vocab"], 43)
        a, b = cpu.forward_chunk(more, len(toks)), gpu.forward_chunk(more, len(toks))
        assert np.array_equal(bits(a), bits(b))
    finally:
        cpu.close()
        gpu.close()


def test_patched_forward_matches_reference_2b_block(amd, orc, patched):
    """One block at BitNet-2B widths (2560 / 6912, 20 x 128 heads, 5 KV
    heads; reduced vocabulary): every projection of the block through the GPU
    row, logits bit for bit."""
    cfg = dict(amd.BITNET_2B, n_layer=1, n_vocab=512)
    model = amd.synth_model(cfg, 44)
    cpu, gpu = _pair(orc, patched, model, 16)
    try:
        for pos, t in enumerate(_tokens(6, cfg["n_vocab"], 45)):
            print(f"[dropin] 2B block: token {pos}", flush=True)
            assert np.array_equal(bits(cpu.forward(t, pos)), bits(gpu.forward(t, pos))), pos
        a = cpu.forward_chunk([3, 4, 5], 6)
        b = gpu.forward_chunk([3, 4, 5], 6)
        assert np.array_equal(bits(a), bits(b))
    finally:
        cpu.close()
        gpu.close()


def test_row_uploads_on_first_gemv_and_releases_with_the_model(amd, orc, patched):
    """The patched load uploads nothing; the first forward step's GEMVs
    upload every I2_S tensor of the model (the row's first whole-matrix
    sllm_gemv); a second model over the same image uses the same copies;
    freeing one model drops the row's copies and the other, still open,
    uploads its tensors again on its next GEMV, its logits still the
    reference's bit for bit; freeing the last leaves nothing on the device."""
    from oracle.gguf_synth import gguf_image
    model = amd.synth_model(TINY, 46)
    image = np.frombuffer(gguf_image(model), np.uint8)
    weights = _weights(amd, image)
    assert len(weights) == 7 * TINY["n_layer"]
    dev_of = amd.lib().sllm_gfx950_tensor_device
    on_device = lambda: [bool(dev_of(ctypes.c_void_p(w))) for w in weights]  # noqa: E731
    assert not any(on_device())
    st = ctypes.c_int()
    r1 = patched.ref_model_open(orc._p(image), image.nbytes, ctypes.byref(st))
    assert r1, st.value
    r2 = c1 = c2 = None
    cpu = orc.RefDecoder(model, 16)
    toks = _tokens(4, TINY["n_vocab"], 47)

    def step(r, c, pos):
        got = np.empty(TINY["n_vocab"], np.float32)
        assert patched.ref_forward(r, c, toks[pos], pos, orc._p(got)) == 0
        return got
    try:
        assert not any(on_device())                  # the load registers nothing
        c1 = patched.ref_ctx_new(r1, 16)
        want0 = cpu.forward(toks[0], 0)
        assert np.array_equal(bits(step(r1, c1, 0)), bits(want0))
        assert all(on_device())                      # the first step's GEMVs uploaded every tensor
        r2 = patched.ref_model_open(orc._p(image), image.nbytes, ctypes.byref(st))
        assert r2, st.value
        c2 = patched.ref_ctx_new(r2, 16)
        assert np.array_equal(bits(step(r2, c2, 0)), bits(want0))
        patched.ref_ctx_free(c1)
        c1 = None
        patched.ref_model_close(r1)
        r1 = None
        assert not any(on_device())                  # freeing a model drops the row's copies
        for pos in range(1, len(toks)):
            assert np.array_equal(bits(step(r2, c2, pos)), bits(cpu.forward(toks[pos], pos))), pos
        assert all(on_device())                      # uploaded again for the model still open
    finally:
        cpu.close()
        for c, r in ((c1, r1), (c2, r2)):
            if c:
                patched.ref_ctx_free(c)
            if r:
                patched.ref_model_close(r)
    assert not any(on_device())

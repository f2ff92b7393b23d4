"""The decode-step oracle, pinned before it is trusted.

Each float operation of the oracle (oracle/sllm_oracle_fwd.c) is checked bit
for bit against the reference's own src/ops.c compiled into oracle/_ref, on
random inputs and on the edges each operation has (scalar tails, the
exponential's out-of-range branches, zeros, subnormals, ties). The whole
decode step is checked against the reference's own sllm_forward
(src/forward.c, loading a GGUF image of the same synthetic model with
src/gguf.c): logits bit for bit, token after token. A planted mistake in a
numpy restatement shows the RMSNorm check can fail.
"""
import ctypes
import os

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
needs_ref = pytest.mark.skipif(
    not os.path.exists(os.path.join(ROOT, "oracle", "_ref", "libsllm_ref.so")),
    reason="oracle/_ref not built (reference tree absent at build time)")

P = lambda a: a.ctypes.data_as(ctypes.c_void_p)
TINY = dict(n_layer=2, n_embd=256, n_ff=512, n_head=4, n_head_kv=2, n_rot=64, n_vocab=1000,
            eps=1e-5, rope_base=500000.0)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_f16_conversion_is_exact_for_every_code(orc):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = np.array([orc.orc().orc_f16_to_f32(int(v)) for v in h], np.float32)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(bits(got)[~nan], bits(want)[~nan])
    assert np.isnan(got[nan]).all()


def test_embedding_conversion_halves_only_subnormals(orc):
    """The token-embedding lookup (src/forward.c:239-262) builds a binary16
    subnormal with an exponent one too low: exactly half the IEEE value. Every
    other code converts exactly. The whole-token checks below against
    sllm_forward fix that this is what the reference does; this fixes that
    nothing else differs."""
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = np.array([orc.orc().orc_f16_to_f32_embd(int(v)) for v in h], np.float32)
    want = h.view(np.float16).astype(np.float32)
    sub = ((h & 0x7C00) == 0) & ((h & 0x3FF) != 0)
    want[sub] *= np.float32(0.5)              # exact: the halves are normal f32
    nan = np.isnan(want)
    assert sub.sum() == 2 * 1023
    assert np.array_equal(bits(got)[~nan], bits(want)[~nan])
    assert np.isnan(got[nan]).all()


@needs_ref
@pytest.mark.parametrize("n", [2560, 6912, 8, 100, 7, 1])
def test_rms_norm_matches_the_reference(orc, n):
    rng = np.random.default_rng(n)
    for trial in range(4):
        x = (rng.standard_normal(n) * rng.uniform(1e-3, 1e3)).astype(np.float32)
        if trial == 3:
            x[::3] = 0.0
        w = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
        for weight in (w, None):
            a, b = np.empty(n, np.float32), np.empty(n, np.float32)
            wp = P(weight) if weight is not None else None
            orc.orc().orc_rms_norm(P(a), P(x), wp, n, 1e-5)
            orc.ref().sllm_rms_norm(P(b), P(x), wp, n, 1e-5)
            assert np.array_equal(bits(a), bits(b))
    # in place, as the FFN sub-norm runs it (src/forward.c:784-786)
    x = rng.standard_normal(n).astype(np.float32)
    a, b = x.copy(), x.copy()
    orc.orc().orc_rms_norm(P(a), P(a), P(w), n, 1e-5)
    orc.ref().sllm_rms_norm(P(b), P(b), P(w), n, 1e-5)
    assert np.array_equal(bits(a), bits(b))
    # all zeros: mean 0, scale 1/sqrt(eps)
    z = np.zeros(n, np.float32)
    a, b = np.empty(n, np.float32), np.empty(n, np.float32)
    orc.orc().orc_rms_norm(P(a), P(z), P(w), n, 1e-5)
    orc.ref().sllm_rms_norm(P(b), P(z), P(w), n, 1e-5)
    assert np.array_equal(bits(a), bits(b))


def _rms_mean(x):
    """The reference's four-lane double sum of f32 squares, narrowed to f32."""
    sq = (x * x).astype(np.float32).astype(np.float64).reshape(-1, 8)
    lanes = [0.0, 0.0, 0.0, 0.0]
    for row in sq:
        for k in range(4):
            lanes[k] += row[k]
        for k in range(4):
            lanes[k] += row[k + 4]
    ss = 0.0
    for k in range(4):
        ss += lanes[k]
    return np.float32(ss / x.size)


def test_rms_norm_restated_and_a_planted_sqrt_mistake_is_caught(orc):
    """A numpy restatement reproduces the oracle; the same restatement with
    the square root taken in double and narrowed (the alternative
    src/ops.c:296-306 warns against) is caught on some vector."""
    rng = np.random.default_rng(3)
    caught = False
    for _ in range(200):
        x = (rng.standard_normal(256) * np.exp(rng.uniform(-4, 4))).astype(np.float32)
        a = np.empty(256, np.float32)
        orc.orc().orc_rms_norm(P(a), P(x), None, 256, 1e-5)
        mean = _rms_mean(x)
        scale = np.float32(1.0) / np.sqrt(mean + np.float32(1e-5), dtype=np.float32)
        assert np.array_equal(bits((scale * x).astype(np.float32)), bits(a))
        planted = np.float32(1.0 / np.sqrt(np.float64(mean + np.float32(1e-5))))
        if not np.array_equal(bits((planted * x).astype(np.float32)), bits(a)):
            caught = True
    assert caught


@needs_ref
@pytest.mark.parametrize("n", [1, 7, 8, 9, 64, 1025, 1031])
def test_softmax_matches_the_reference(orc, n):
    rng = np.random.default_rng(n + 100)
    for spread in (1.0, 30.0, 500.0):
        x = (rng.standard_normal(n) * spread).astype(np.float32)
        a, b = x.copy(), x.copy()
        orc.orc().orc_softmax(P(a), n)
        orc.ref().sllm_softmax_inplace(P(b), n)
        assert np.array_equal(bits(a), bits(b)), spread


@needs_ref
@pytest.mark.parametrize("n", [6912, 13, 8])
def test_silu_matches_the_reference(orc, n):
    rng = np.random.default_rng(n + 7)
    for spread in (1.0, 40.0, 300.0):
        x = (rng.standard_normal(n) * spread).astype(np.float32)
        a, b = x.copy(), x.copy()
        orc.orc().orc_silu(P(a), n)
        orc.ref().sllm_silu_inplace(P(b), n)
        assert np.array_equal(bits(a), bits(b)), spread


def test_v_expf_covers_its_three_ranges(orc):
    """Arguments whose rounded exponent stays within 126, goes past it and
    past 192 (the blend's branches), each against exp to within a few ulp."""
    for x in (-3.5, 0.0, 1.0, 80.0, -87.0, 88.5, -100.0, -140.0, 200.0, -200.0):
        got = orc.orc().orc_v_expf(x)
        want = np.exp(np.float64(x))
        if want > 3.4e38:
            assert np.isinf(got)
        elif want < 1e-45:
            assert got == 0.0
        else:
            assert abs(got - want) <= 4 * np.spacing(np.float32(want)) + 1e-45, x


@needs_ref
def test_rope_matches_the_reference(orc):
    rng = np.random.default_rng(9)
    for n_rot in (128, 64, 7):
        for pos in (0, 1, 17, 1024, 4095, 30000):
            x = rng.standard_normal(128).astype(np.float32) * 50
            a, b = x.copy(), x.copy()
            orc.orc().orc_rope_neox(P(a), n_rot, pos, 500000.0, 1.0)
            orc.ref().sllm_rope_inplace(P(b), n_rot, pos, 500000.0, 1.0, 0)   # SLLM_ROPE_NEOX
            assert np.array_equal(bits(a), bits(b)), (n_rot, pos)
            # the cos / sin table form gives the same rotation
            half = (n_rot - n_rot % 2) // 2
            cs, sn = np.empty(half, np.float32), np.empty(half, np.float32)
            orc.orc().orc_rope_cos_sin(n_rot, pos, 500000.0, 1.0, P(cs), P(sn))
            c = x.copy()
            xa, xb = c[:half].copy(), c[half:2 * half].copy()
            c[:half] = xa * cs - xb * sn
            c[half:2 * half] = xa * sn + xb * cs
            assert np.array_equal(bits(c), bits(a)), (n_rot, pos)


@needs_ref
@pytest.mark.parametrize("n", [2560, 32, 100, 5])
def test_f16_dot_matches_the_reference(orc, n):
    rng = np.random.default_rng(n + 3)
    for _ in range(6):
        row = rng.standard_normal(n).astype(np.float16)
        row[rng.integers(0, n, 2)] = np.float16(3e-6)          # binary16 subnormals
        x = (rng.standard_normal(n) * 30).astype(np.float32)
        h = row.view(np.uint16)
        assert orc.orc().orc_dot_f16(P(h), P(x), n) == orc.ref().sllm_dot_f16_f32(P(h), P(x), n)
        got = np.float32(orc.orc().orc_dot_f16(P(h), P(x), n))
        want = np.float32(orc.ref().sllm_dot_f16_f32(P(h), P(x), n))
        assert got.tobytes() == want.tobytes()


@needs_ref
def test_argmax_matches_the_reference(orc):
    cases = [np.array([1, 3, 3, 2], np.float32), np.array([np.nan, 5, 6], np.float32),
             np.array([0.0, -0.0, 0.0], np.float32), np.array([-np.inf, -np.inf], np.float32),
             np.array([2, np.nan, 7, 7], np.float32),
             np.random.default_rng(0).standard_normal(128256).astype(np.float32)]
    for c in cases:
        assert orc.orc().orc_argmax(P(c), c.size) == orc.ref().ref_argmax(P(c), c.size)


def _tokens(n, vocab, seed):
    return [int(t) for t in np.random.default_rng(seed).integers(0, vocab, n)]


@needs_ref
@pytest.mark.parametrize("cfg", [
    TINY,
    dict(TINY, n_layer=3, n_embd=512, n_ff=1024, n_head=8, n_head_kv=2, n_rot=48, n_vocab=777),
])
def test_decode_step_matches_the_reference_forward(amd, orc, cfg):
    """Token after token from position 0 (softmax with and without scalar
    tails), logits bit for bit against the reference's own sllm_forward on a
    GGUF image of the same model."""
    model = amd.synth_model(cfg, 3)
    tokens = _tokens(20, cfg["n_vocab"], 5)
    # binary16 subnormals (and a negative one) in the rows looked up, so the
    # embedding conversion's halving is on the path at several positions
    emb = np.asarray(model["tok_embd"]).reshape(cfg["n_vocab"], cfg["n_embd"])
    for i, t in enumerate(tokens[::3]):
        emb[t, (7 * i) % cfg["n_embd"]] = (0x0001, 0x03FF, 0x8200, 0x0155)[i % 4]
    d, r = orc.Decoder(model, 40), orc.RefDecoder(model, 40, threads=4)
    try:
        for pos, tok in enumerate(tokens):
            a = d.forward(tok, pos)
            b = r.forward(tok, pos)
            assert np.array_equal(bits(a), bits(b)), pos
            assert orc.orc().orc_argmax(P(a), a.size) == orc.ref().ref_argmax(P(b), b.size)
    finally:
        d.close()
        r.close()


@needs_ref
def test_decode_step_at_bitnet_2b_widths(amd, orc):
    """One layer at the real widths (2560 / 6912, 20 x 128 heads, 5 KV heads)
    with a reduced vocabulary: the same bits as the reference's forward."""
    cfg = dict(amd.BITNET_2B, n_layer=1, n_vocab=512)
    model = amd.synth_model(cfg, 4)
    d, r = orc.Decoder(model, 16), orc.RefDecoder(model, 16, threads=4)
    try:
        for pos, tok in enumerate(_tokens(10, cfg["n_vocab"], 6)):
            logits, dots, acts = d.forward(tok, pos, trace=True)
            assert np.array_equal(bits(logits), bits(r.forward(tok, pos))), pos
            assert dots.size == orc.n_trace_dots(cfg) and np.abs(dots).max() > 0
            assert (acts["scale"] > 0).all()
    finally:
        d.close()
        r.close()


@needs_ref
def test_state_file_restores_the_reference_cache(amd, orc, tmp_path):
    """A cache prefix handed to the reference through its own state file
    (src/forward.c:963-1100) and the same prefix written into the oracle's
    cache: the next tokens' logits agree bit for bit -- the layout both use,
    [layer][head_kv][pos][head_dim], and the position after the prefix."""
    from oracle.gguf_synth import state_image
    cfg = dict(TINY, n_layer=2)
    model = amd.synth_model(cfg, 13)
    rng = np.random.default_rng(14)
    hd = cfg["n_embd"] // cfg["n_head"]
    shape = (cfg["n_layer"], cfg["n_head_kv"], 100, hd)
    k = rng.standard_normal(shape).astype(np.float16).astype(np.float32)
    v = rng.standard_normal(shape).astype(np.float16).astype(np.float32)
    path = tmp_path / "prefix.slkv"
    path.write_bytes(state_image(cfg, 128, k, v, np.zeros(cfg["n_vocab"], np.float32)))
    r, d = orc.RefDecoder(model, 128, threads=2), orc.Decoder(model, 128)
    try:
        r.state_load(str(path))
        ok, ov = d.caches()
        ok[:, :, :100] = k
        ov[:, :, :100] = v
        for i, tok in enumerate(_tokens(4, cfg["n_vocab"], 15)):
            assert np.array_equal(bits(r.forward(tok, 100 + i)), bits(d.forward(tok, 100 + i))), i
    finally:
        r.close()
        d.close()


@needs_ref
def test_reference_chunks_equal_its_token_path_and_the_oracle(amd, orc):
    """sllm_forward_chunk / sllm_forward_prefill_chunked of the reference
    (src/forward.c:589-868) give every position's logits bit for bit as its
    one-token forward does (the property tests/test_phase5.c:85-150 of the
    reference asserts), and those are the oracle's token-by-token logits: the
    target a device chunk is checked against. Chunk sizes below, at and above
    the sequence; a later chunk attends to keys an earlier one wrote."""
    cfg = dict(TINY, n_layer=2)
    model = amd.synth_model(cfg, 17)
    toks = _tokens(19, cfg["n_vocab"], 18)
    d = orc.Decoder(model, 32)
    try:
        want = np.stack([d.forward(t, p) for p, t in enumerate(toks)])
    finally:
        d.close()
    for chunk in (1, 2, 5, 19, 32):
        r = orc.RefDecoder(model, 32, threads=2)
        try:
            got = r.prefill_chunked(toks, chunk)
        finally:
            r.close()
        assert np.array_equal(bits(got), bits(want)), f"chunk {chunk}"
    r = orc.RefDecoder(model, 32, threads=2)
    try:
        a = r.forward_chunk(toks[:7], 0)
        b = r.forward_chunk(toks[7:], 7)
    finally:
        r.close()
    assert np.array_equal(bits(np.concatenate([a, b])), bits(want))

"""Chunks of tokens on the GPU (sllm_gfx950_forward_chunk,
sllm_gfx950_forward_prefill_chunked) against the oracle.

The reference's chunk path gives every position the logits of its one-token
path bit for bit (tests/test_oracle_fwd.py runs its own
sllm_forward_prefill_chunked to show it), and the oracle's token-by-token
logits are those bits; so every row of a device chunk must equal the
oracle's logits at that position, bit for bit. Shapes: chunk sizes from 2
to 64 over a 70-token sequence (later chunks attend to keys earlier ones
wrote), chunks over a restored 1024-position cache at tiny and BitNet-2B
widths, chunks of 200 and 150 tokens (the scores' eight-token workgroups),
the full 30-block 2B model in one 100-token chunk, 512-token chunks at 2B
widths, the cache store folded into the Q + K + V GEMM (forced tiles),
widths where no GEMM epilogue is fused (384 / 640), and decode / greedy
generation carrying on after a chunk.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TINY = dict(n_layer=2, n_embd=256, n_ff=512, n_head=4, n_head_kv=2, n_rot=64, n_vocab=1000,
            eps=1e-5, rope_base=500000.0)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _tokens(n, vocab, seed):
    return [int(t) for t in np.random.default_rng(seed).integers(0, vocab, n)]


def _oracle_logits(orc, model, n_ctx, toks, base=0, caches=None):
    o = orc.Decoder(model, n_ctx)
    try:
        if caches is not None:
            ok, ov = o.caches()
            k, v = caches
            ok[:, :, :k.shape[2]] = k
            ov[:, :, :v.shape[2]] = v
        return np.stack([o.forward(t, base + p) for p, t in enumerate(toks)])
    finally:
        o.close()


def _first_diff(got, want):
    bad = np.argwhere(bits(got) != bits(want))
    return f"first differing (position, row) {tuple(bad[0])} of {len(bad)}" if len(bad) else ""


@pytest.fixture(scope="module")
def tiny(amd, orc):
    model = amd.synth_model(TINY, 71)
    toks = _tokens(70, TINY["n_vocab"], 72)
    emb = np.asarray(model["tok_embd"]).reshape(TINY["n_vocab"], TINY["n_embd"])
    for i, t in enumerate(toks[::5]):                 # binary16 subnormals in the lookup
        emb[t, (11 * i) % TINY["n_embd"]] = (0x0001, 0x03FF, 0x8200, 0x0155)[i % 4]
    return model, toks, _oracle_logits(orc, model, 80, toks)


@pytest.mark.parametrize("chunk", [2, 3, 7, 16, 64])
def test_chunked_prefill_matches_token_by_token(amd, dev, tiny, chunk):
    model, toks, want = tiny
    print(f"[chunk] prefill 70 tokens in chunks of {chunk}", flush=True)
    g = amd.DeviceDecoder(dev, model, 80)
    try:
        got = g.prefill_chunked(toks, chunk)
        assert g.n_past() == len(toks)
    finally:
        g.close()
    assert np.array_equal(bits(got), bits(want)), _first_diff(got, want)


def test_chunks_at_uneven_positions_then_decode(amd, dev, tiny):
    """forward_chunk at base 0 (5 tokens), a single token, a chunk of 30, then
    one token at a time; the graph-replayed decode step carries on from the
    cache the chunks wrote."""
    model, toks, want = tiny
    g = amd.DeviceDecoder(dev, model, 80)
    g.set_graph(True)
    try:
        rows = [g.forward_chunk(toks[:5], 0), g.forward_chunk(toks[5:6], 5), g.forward_chunk(toks[6:36], 6)]
        rows += [g.forward(t, p)[None] for p, t in enumerate(toks[36:45], 36)]
        rows.append(g.forward_chunk(toks[45:70], 45))
        got = np.concatenate(rows)
    finally:
        g.close()
    assert np.array_equal(bits(got), bits(want)), _first_diff(got, want)


def test_chunk_without_logits_keeps_the_last_and_greedy_continues(amd, orc, dev, tiny):
    """logits = NULL: the output head runs for the last token only; its
    argmax starts a greedy continuation, as after a one-token forward."""
    model, toks, want = tiny
    g = amd.DeviceDecoder(dev, model, 80)
    u = amd.DeviceDecoder(dev, model, 80)
    try:
        assert g.forward_chunk(toks[:40], 0, logits=False) is None
        assert g.argmax() == int(np.argmax(want[39]))
        for p, t in enumerate(toks[:40]):
            u.forward(t, p, logits=False)
        assert np.array_equal(g.generate([], 12), u.generate([], 12))
    finally:
        g.close()
        u.close()


def test_chunks_with_a_narrow_rotary_width_and_four_query_heads_per_kv_head(amd, orc, dev):
    """n_rot 48 of a 64-wide head (dimensions 48..63 pass through RoPE),
    eight query heads over two KV heads: prefill in chunks of 5 and 23,
    every position's logits against the oracle."""
    cfg = dict(TINY, n_layer=3, n_embd=512, n_ff=1024, n_head=8, n_head_kv=2, n_rot=48, n_vocab=777)
    model = amd.synth_model(cfg, 78)
    toks = _tokens(51, cfg["n_vocab"], 79)
    want = _oracle_logits(orc, model, 64, toks)
    print("[chunk] narrow rotary width, 4 query heads per KV head", flush=True)
    for chunk in (5, 23):
        g = amd.DeviceDecoder(dev, model, 64)
        try:
            got = g.prefill_chunked(toks, chunk)
        finally:
            g.close()
        assert np.array_equal(bits(got), bits(want)), f"chunk {chunk}: " + _first_diff(got, want)


def test_chunks_above_128_tokens(amd, orc, dev):
    """A chunk of 200 tokens, then one of 150 at positions 200..349: above
    128 tokens the scores take eight tokens per workgroup, and the second
    chunk's rows run past 256 positions; every position's logits against
    the oracle."""
    cfg = dict(TINY, n_layer=2)
    model = amd.synth_model(cfg, 81)
    toks = _tokens(350, cfg["n_vocab"], 82)
    want = _oracle_logits(orc, model, 360, toks)
    print("[chunk] 200 + 150 tokens", flush=True)
    g = amd.DeviceDecoder(dev, model, 360)
    try:
        got = np.concatenate([g.forward_chunk(toks[:200], 0), g.forward_chunk(toks[200:], 200)])
    finally:
        g.close()
    assert np.array_equal(bits(got), bits(want)), _first_diff(got, want)


def test_chunks_where_no_gemm_epilogue_is_fused(amd, orc, dev):
    """Widths that are multiples of 128 but not of 256 (n_embd 384, n_ff
    640): every projection takes the split-K tiles, which have no fused
    epilogue, so the chunk runs its own cache store, SiLU and residual sums
    (the 256-multiple widths of the other tests take the fused forms);
    prefill in chunks of 7 and 100 tokens (the tiles on either side of 64),
    every position's logits against the oracle."""
    cfg = dict(TINY, n_layer=3, n_embd=384, n_ff=640, n_head=6, n_head_kv=2, n_rot=64, n_vocab=555)
    model = amd.synth_model(cfg, 86)
    toks = _tokens(140, cfg["n_vocab"], 87)
    want = _oracle_logits(orc, model, 160, toks)
    print("[chunk] widths 384 / 640: no fused GEMM epilogue", flush=True)
    for chunk in (7, 100):
        g = amd.DeviceDecoder(dev, model, 160)
        try:
            got = g.prefill_chunked(toks, chunk)
        finally:
            g.close()
        assert np.array_equal(bits(got), bits(want)), f"chunk {chunk}: " + _first_diff(got, want)


def _prefix_case(amd, orc, dev, widths):
    cfg = dict(TINY) if widths == "tiny" else dict(amd.BITNET_2B, n_layer=2, n_vocab=512)
    model = amd.synth_model(cfg, 73)
    n_pos, n_ctx = 1024, 1072
    hd = cfg["n_embd"] // cfg["n_head"]
    rng = np.random.default_rng(74)
    shape = (cfg["n_layer"], cfg["n_head_kv"], n_pos, hd)
    k = rng.standard_normal(shape).astype(np.float16).astype(np.float32)
    v = rng.standard_normal(shape).astype(np.float16).astype(np.float32)
    toks = _tokens(40, cfg["n_vocab"], 75)
    want = _oracle_logits(orc, model, n_ctx, toks, n_pos, (k, v))
    print(f"[chunk] {widths}: 40 tokens after a {n_pos}-position prefix", flush=True)
    g = amd.DeviceDecoder(dev, model, n_ctx)
    try:
        g.kv_load(k, v, n_pos)
        got = np.concatenate([g.forward_chunk(toks[:24], n_pos), g.forward_chunk(toks[24:], n_pos + 24)])
    finally:
        g.close()
    assert np.array_equal(bits(got), bits(want)), _first_diff(got, want)


@pytest.mark.parametrize("widths", ["tiny", "2b"])
def test_chunk_over_a_1024_position_prefix(amd, orc, dev, widths):
    """40 tokens at positions 1024..1063 over a restored cache: every query's
    softmax spans its own KV rows past the prefix."""
    _prefix_case(amd, orc, dev, widths)


@pytest.mark.parametrize("tile", [10, 13])
def test_cache_store_in_the_qkv_epilogue(amd, orc, dev, tiny, tile):
    """Where the Q + K + V GEMM's row tiles hold whole heads (the 64 x 256 and
    32 x 128 tiles, forced here: set_gemm_tile 10 and 13) its epilogue ropes
    the queries and writes the keys and values into the caches itself, in
    place of sllm_k_chk_kv_store. Forced at sizes where the automatic choice
    takes other tiles: the tiny model in chunks of 7 and 64 (two or four
    64-wide heads per tile, K and V tiles past their 128 rows), the narrow
    rotary width (n_rot 48 of 64), 2B widths over a 1024-position cache
    (one or two 128-wide heads per tile); then greedy decoding from the
    caches the chunks wrote, against token-by-token decoding."""
    model, toks, want = tiny
    print(f"[chunk] cache store in the QKV epilogue, tile {tile}", flush=True)
    dev.set_gemm_tile(tile)
    try:
        for chunk in (7, 64):
            g = amd.DeviceDecoder(dev, model, 80)
            try:
                got = g.prefill_chunked(toks, chunk)
            finally:
                g.close()
            assert np.array_equal(bits(got), bits(want)), f"chunk {chunk}: " + _first_diff(got, want)
        cfg = dict(TINY, n_layer=3, n_embd=512, n_ff=1024, n_head=8, n_head_kv=2, n_rot=48, n_vocab=777)
        m2 = amd.synth_model(cfg, 78)
        t2 = _tokens(51, cfg["n_vocab"], 79)
        w2 = _oracle_logits(orc, m2, 64, t2)
        g = amd.DeviceDecoder(dev, m2, 64)
        try:
            got = g.prefill_chunked(t2, 23)
        finally:
            g.close()
        assert np.array_equal(bits(got), bits(w2)), "narrow rotary: " + _first_diff(got, w2)
        _prefix_case(amd, orc, dev, "2b")
        g = amd.DeviceDecoder(dev, model, 80)
        u = amd.DeviceDecoder(dev, model, 80)
        try:
            assert g.forward_chunk(toks[:40], 0, logits=False) is None
            for p, t in enumerate(toks[:40]):
                u.forward(t, p, logits=False)
            assert np.array_equal(g.generate([], 12), u.generate([], 12))
        finally:
            g.close()
            u.close()
    finally:
        dev.set_gemm_tile(0)


def test_full_2b_chunk_is_bit_exact(amd, orc, dev):
    """All 30 blocks at BitNet-2B shape, 100 tokens in one chunk (every GEMM
    on a direct-load MFMA tile), logits of every position against the oracle."""
    cfg = dict(amd.BITNET_2B)
    print("[chunk] building the 2B model", flush=True)
    model = amd.synth_model(cfg, 5)
    toks = _tokens(100, cfg["n_vocab"], 76)
    print("[chunk] oracle, 100 tokens", flush=True)
    want = _oracle_logits(orc, model, 128, toks)
    g = amd.DeviceDecoder(dev, model, 128)
    try:
        print("[chunk] device chunk of 100", flush=True)
        got = g.forward_chunk(toks, 0)
    finally:
        g.close()
    assert np.array_equal(bits(got), bits(want)), _first_diff(got, want)


@pytest.mark.parametrize("prefix", [0, 1024])
def test_2b_width_512_token_chunk_every_position(amd, orc, dev, prefix):
    """One chunk of 512 tokens -- the device's largest, twice the reference's
    cap -- at BitNet-2B widths (20 x 128 query heads over 5 KV heads, FFN
    6912; two blocks and a 512-row vocabulary keep the oracle to seconds),
    from position 0 as the prefill benchmark runs it, and after a restored
    1024-position cache (rows up to 1536 positions). Every token's scores
    workgroup of eight, every p.V chain length from 1 to 512 (and 1025 to
    1536): every position's logits against the oracle's token-by-token
    logits, bit for bit."""
    cfg = dict(amd.BITNET_2B, n_layer=2, n_vocab=512)
    model = amd.synth_model(cfg, 93)
    toks = _tokens(512, cfg["n_vocab"], 94 + prefix)
    n_ctx = prefix + 512 + 8
    caches = None
    if prefix:
        hd = cfg["n_embd"] // cfg["n_head"]
        rng = np.random.default_rng(95)
        shape = (cfg["n_layer"], cfg["n_head_kv"], prefix, hd)
        caches = (rng.standard_normal(shape).astype(np.float16).astype(np.float32),
                  rng.standard_normal(shape).astype(np.float16).astype(np.float32))
    print(f"[chunk] 2B widths: oracle, 512 tokens after {prefix} positions", flush=True)
    want = _oracle_logits(orc, model, n_ctx, toks, prefix, caches)
    g = amd.DeviceDecoder(dev, model, n_ctx)
    try:
        if caches is not None:
            g.kv_load(caches[0], caches[1], prefix)
        print("[chunk] device chunk of 512", flush=True)
        got = g.forward_chunk(toks, prefix)
        assert g.n_past() == prefix + 512
    finally:
        g.close()
    assert np.array_equal(bits(got), bits(want)), _first_diff(got, want)


def test_chunk_refuses_what_the_reference_refuses(amd, dev):
    cfg = dict(TINY, n_layer=1)
    model = amd.synth_model(cfg, 77)
    g = amd.DeviceDecoder(dev, model, 600)
    try:
        assert g.status_chunk([], 0) == -1                           # n < 1
        assert g.status_chunk([1] * 513, 0) == -1                    # n above the limit
        assert g.status_chunk([1, cfg["n_vocab"]], 0) == -1          # token out of range
        assert g.status_chunk([1, -1], 0) == -1
        assert g.status_chunk([1, 2], 599) == -1                     # past n_ctx
        assert g.status_chunk([1, 2, 3], 4) == 0                     # a gap is allowed
        assert g.n_past() == 7
        assert g.status_chunk([1, 2], 6) == -1                       # rewinding is not
        assert g.status_prefill([1, 2], 2) == -1                     # prefill starts at 0: rewinds
        g.reset()
        assert g.status_prefill([1, 2], 0) == -1                     # chunk 0
        assert g.status_prefill([1, 2], 513) == -1                   # chunk above the limit
        assert g.status_prefill([1] * 601, 4) == -36                 # more tokens than n_ctx
        assert g.status_prefill([1] * 512, 512) == 0
        assert g.n_past() == 512
    finally:
        g.close()

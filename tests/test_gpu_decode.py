"""The decode step on the GPU (sllm_gfx950_decode.h) against the oracle.

The oracle's decode step is pinned bit for bit to the reference's own
sllm_forward (tests/test_oracle_fwd.py), so agreement here is agreement
with the reference: logits bit for bit, token after token, and -- through
the trace -- every projection's int32 dots and every activation's scale /
sum. Shapes: tiny models (every position from 0, scalar softmax tails of
every length, a rotary width below the head width, four query heads per KV
head), one block at BitNet-2B widths, a 1024-position KV prefix holding
binary16 values, and the full 30-block 2B shape.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TINY = dict(n_layer=2, n_embd=256, n_ff=512, n_head=4, n_head_kv=2, n_rot=64, n_vocab=1000,
            eps=1e-5, rope_base=500000.0)
NARROW_ROT = dict(TINY, n_layer=3, n_embd=512, n_ff=1024, n_head=8, n_head_kv=2, n_rot=48, n_vocab=777)


def cfg_label(cfg):
    return f"{cfg['n_layer']}x{cfg['n_embd']}/{cfg['n_ff']} h{cfg['n_head']}/{cfg['n_head_kv']} rot{cfg['n_rot']}"


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _tokens(n, vocab, seed):
    return [int(t) for t in np.random.default_rng(seed).integers(0, vocab, n)]


def _plant_subnormals(model, tokens):
    cfg = model["cfg"]
    emb = np.asarray(model["tok_embd"]).reshape(cfg["n_vocab"], cfg["n_embd"])
    for i, t in enumerate(tokens[::3]):
        emb[t, (7 * i) % cfg["n_embd"]] = (0x0001, 0x03FF, 0x8200, 0x0155)[i % 4]


def _compare_step(g, o, tok, pos, label):
    want, wdots, wacts = o.forward(tok, pos, trace=True)
    got = g.forward(tok, pos)
    gdots, gacts = g.trace_read()
    assert np.array_equal(gdots, wdots), f"{label}: int32 dots differ at pos {pos}"
    assert np.array_equal(gacts["sum"], wacts["sum"]), f"{label}: act sums differ at pos {pos}"
    assert np.array_equal(bits(gacts["scale"]), bits(wacts["scale"])), f"{label}: act scales differ at pos {pos}"
    assert np.array_equal(bits(got), bits(want)), f"{label}: logits differ at pos {pos}"


@pytest.mark.parametrize("cfg", [TINY, NARROW_ROT], ids=["tiny", "narrow-rot"])
def test_decode_matches_the_oracle_token_by_token(amd, orc, dev, cfg):
    model = amd.synth_model(cfg, 3)
    tokens = _tokens(20, cfg["n_vocab"], 5)
    _plant_subnormals(model, tokens)
    print(f"[decode] {cfg['n_layer']} blocks, {len(tokens)} tokens", flush=True)
    g, o = amd.DeviceDecoder(dev, model, 40), orc.Decoder(model, 40)
    g.trace_start()
    try:
        for pos, tok in enumerate(tokens):
            _compare_step(g, o, tok, pos, cfg_label(cfg))
    finally:
        g.trace_stop()
        g.close()
        o.close()


def test_argmax_follows_the_first_maximum(amd, orc, dev):
    cfg = dict(TINY, n_layer=1)
    model = amd.synth_model(cfg, 8)
    g, o = amd.DeviceDecoder(dev, model, 16), orc.Decoder(model, 16)
    try:
        for pos, tok in enumerate(_tokens(6, cfg["n_vocab"], 9)):
            want = o.forward(tok, pos)
            g.forward(tok, pos, logits=False)
            assert g.argmax() == orc.orc().orc_argmax(orc._p(want), cfg["n_vocab"])
    finally:
        g.close()
        o.close()


def test_one_block_at_bitnet_2b_widths(amd, orc, dev):
    cfg = dict(amd.BITNET_2B, n_layer=1, n_vocab=512)
    model = amd.synth_model(cfg, 4)
    print("[decode] one 2B block", flush=True)
    g, o = amd.DeviceDecoder(dev, model, 16), orc.Decoder(model, 16)
    g.trace_start()
    try:
        for pos, tok in enumerate(_tokens(10, cfg["n_vocab"], 6)):
            _compare_step(g, o, tok, pos, "2b-block")
    finally:
        g.trace_stop()
        g.close()
        o.close()


def _kv_prefix(cfg, n_pos, seed):
    """f32 caches [layer][head_kv][pos][head_dim] of binary16 N(0,1) values."""
    hd = cfg["n_embd"] // cfg["n_head"]
    shape = (cfg["n_layer"], cfg["n_head_kv"], n_pos, hd)
    rng = np.random.default_rng(seed)
    k = rng.standard_normal(shape).astype(np.float16).astype(np.float32)
    v = rng.standard_normal(shape).astype(np.float16).astype(np.float32)
    return k, v


@pytest.mark.parametrize("widths,n_pos", [("tiny", 1024), ("2b", 1024), ("tiny", 4030)])
def test_decode_after_a_restored_prefix(amd, orc, dev, widths, n_pos):
    """Positions past a restored cache. At 1024 the softmax spans seventeen
    score workgroups per KV head and p.V keeps p and V of the row in one
    round (1536 positions); at 4030 .. 4034 p.V takes three rounds, e
    recomputed for the second and third."""
    cfg = dict(TINY) if widths == "tiny" else dict(amd.BITNET_2B, n_layer=2, n_vocab=512)
    model = amd.synth_model(cfg, 12)
    n_ctx = n_pos + 8
    k, v = _kv_prefix(cfg, n_pos, 13)
    g, o = amd.DeviceDecoder(dev, model, n_ctx), orc.Decoder(model, n_ctx)
    ok, ov = o.caches()
    ok[:, :, :n_pos] = k
    ov[:, :, :n_pos] = v
    g.kv_load(k, v, n_pos)
    assert g.n_past() == n_pos
    g.trace_start()
    print(f"[decode] {widths}: prefix {n_pos}", flush=True)
    try:
        for i, tok in enumerate(_tokens(5, cfg["n_vocab"], 14)):
            _compare_step(g, o, tok, n_pos + i, f"prefix-{widths}")
    finally:
        g.trace_stop()
        g.close()
        o.close()


def _oracle_greedy(o, prompt, n_new, n_vocab):
    from oracle import oracle as orcmod
    pos = 0
    logits = None
    for t in prompt:
        logits = o.forward(t, pos)
        pos += 1
    out = []
    nxt = orcmod.orc().orc_argmax(orcmod._p(logits), n_vocab)
    for _ in range(n_new):
        out.append(nxt)
        logits = o.forward(nxt, pos)
        pos += 1
        nxt = orcmod.orc().orc_argmax(orcmod._p(logits), n_vocab)
    return out, logits


@pytest.mark.parametrize("graph", [False, True], ids=["launches", "graph"])
def test_greedy_generation_runs_on_the_device(amd, orc, dev, graph):
    """The token loop with no host round trip per token: the output kernel
    feeds each argmax back. Same ids as the oracle's loop, and the last
    logits are the oracle's last logits."""
    cfg = dict(NARROW_ROT, n_layer=2)
    model = amd.synth_model(cfg, 21)
    prompt = _tokens(5, cfg["n_vocab"], 22)
    g, o = amd.DeviceDecoder(dev, model, 64), orc.Decoder(model, 64)
    g.set_graph(graph)
    try:
        got = g.generate(prompt, 12)
        want, last = _oracle_greedy(o, prompt, 12, cfg["n_vocab"])
        assert list(got) == want
        assert g.n_past() == len(prompt) + 12
        dl = amd.lib().sllm_gfx950_ctx_logits(g.c)
        dev.sync()
        glast = np.empty(cfg["n_vocab"], np.float32)
        amd.check(amd.lib().sllm_gfx950_d2h(amd.ptr(glast), dl, glast.nbytes))
        assert np.array_equal(bits(glast), bits(last))
        # no prompt: continue from the last logits (src/forward.c:910-919)
        more = g.generate([], 4)
        want2 = []
        nxt = orc.orc().orc_argmax(orc._p(last), cfg["n_vocab"])
        pos = len(prompt) + 12
        for _ in range(4):
            want2.append(nxt)
            lg = o.forward(nxt, pos)
            pos += 1
            nxt = orc.orc().orc_argmax(orc._p(lg), cfg["n_vocab"])
        assert list(more) == want2
    finally:
        g.close()
        o.close()


def test_graph_replays_match_launches(amd, dev):
    cfg = dict(TINY, n_layer=2)
    model = amd.synth_model(cfg, 31)
    toks = _tokens(12, cfg["n_vocab"], 32)
    a, b = amd.DeviceDecoder(dev, model, 16), amd.DeviceDecoder(dev, model, 16)
    b.set_graph(True)
    try:
        for pos, t in enumerate(toks):
            x = a.forward(t, pos)
            y = b.forward(t, pos)
            assert np.array_equal(bits(x), bits(y)), pos
    finally:
        a.close()
        b.close()


def test_forward_refuses_what_the_reference_refuses(amd, dev):
    cfg = dict(TINY, n_layer=1)
    model = amd.synth_model(cfg, 41)
    g = amd.DeviceDecoder(dev, model, 8)
    try:
        assert g.status_forward(cfg["n_vocab"], 0) == -1          # token out of range
        assert g.status_forward(-1, 0) == -1
        assert g.status_forward(1, 8) == -1                       # past n_ctx
        g.forward(1, 0, logits=False)
        g.forward(2, 3, logits=False)                             # a gap is allowed
        assert g.status_forward(3, 2) == -1                       # rewinding is not
        out = np.zeros(8, np.int32)
        st = amd.lib().sllm_gfx950_generate_greedy(g.m, g.c, None, 0, 8, amd.ptr(out))
        assert st == -36                                          # past n_ctx
        g.reset()
        assert g.n_past() == 0
        g.forward(5, 0, logits=False)
    finally:
        g.close()


def test_reset_gives_a_fresh_context(amd, orc, dev):
    cfg = dict(TINY, n_layer=2)
    model = amd.synth_model(cfg, 51)
    toks = _tokens(6, cfg["n_vocab"], 52)
    g = amd.DeviceDecoder(dev, model, 16)
    try:
        first = [g.forward(t, p) for p, t in enumerate(toks)]
        g.reset()
        again = [g.forward(t, p) for p, t in enumerate(toks)]
        for a, b in zip(first, again):
            assert np.array_equal(bits(a), bits(b))
    finally:
        g.close()


def test_a_gguf_model_decodes_like_the_uploaded_one(amd, orc, dev, tmp_path):
    """sllm_gfx950_model_load_gguf (an image) and _file (a path) on the GGUF
    the reference loads: logits bit for bit with the oracle, and greedy
    tokens the same as the uploaded model's."""
    from oracle import gguf_synth
    cfg = dict(TINY, n_layer=2)
    model = amd.synth_model(cfg, 61)
    toks = _tokens(8, cfg["n_vocab"], 62)
    _plant_subnormals(model, toks)
    image = gguf_synth.gguf_image(model)
    path = tmp_path / "tiny.gguf"
    path.write_bytes(image)
    print("[decode] gguf image and file", flush=True)
    a = amd.DeviceDecoder(dev, None, 24, gguf=image)
    b = amd.DeviceDecoder(dev, None, 24, gguf=str(path))
    u = amd.DeviceDecoder(dev, model, 24)
    o = orc.Decoder(model, 24)
    try:
        assert a.cfg["n_layer"] == 2 and b.cfg["n_vocab"] == cfg["n_vocab"]
        for pos, t in enumerate(toks):
            want = o.forward(t, pos)
            for g, label in ((a, "image"), (b, "file")):
                assert np.array_equal(bits(g.forward(t, pos)), bits(want)), f"{label}: logits differ at pos {pos}"
        a.reset()
        u.reset()
        assert np.array_equal(a.generate(toks[:3], 10), u.generate(toks[:3], 10))
    finally:
        for g in (a, b, u, o):
            g.close()


def test_full_2b_decode_is_bit_exact(amd, orc, dev):
    """All 30 blocks at BitNet-2B shape with the 128256-row F16 output: every
    int32 accumulator, every activation and the logits of three tokens."""
    cfg = dict(amd.BITNET_2B)
    print("[decode] building the 2B model", flush=True)
    model = amd.synth_model(cfg, 1)
    g, o = amd.DeviceDecoder(dev, model, 8), orc.Decoder(model, 8)
    g.trace_start()
    try:
        for pos, tok in enumerate(_tokens(3, cfg["n_vocab"], 2)):
            print(f"[decode] 2B token {pos}", flush=True)
            _compare_step(g, o, tok, pos, "2b")
    finally:
        g.trace_stop()
        g.close()
        o.close()


def test_kv_load_restores_a_state_like_the_reference(amd, orc, dev):
    """sllm_gfx950_ctx_kv_load against sllm_state_load (src/forward.c:1040-1121)
    on a context that has already decoded past 1024 positions: the restored
    512-position prefix, zeros from there on in every (layer, KV head) -- a
    forward at a gapped position reads them as the reference does -- and the
    restored last logits, whose argmax an empty-prompt generate continues
    from (src/forward.c:909-912). Without logits, an empty-prompt generate
    is refused until a forward."""
    cfg = dict(TINY, n_layer=2)
    model = amd.synth_model(cfg, 71)
    n_ctx, n_pos, gap = 1100, 512, 700
    g = amd.DeviceDecoder(dev, model, n_ctx)
    print("[decode] kv_load after 1030 positions", flush=True)
    try:
        g.generate(_tokens(6, cfg["n_vocab"], 72), 1024)          # stale rows up to position 1029
        assert g.n_past() == 1030
        k, v = _kv_prefix(cfg, n_pos, 73)
        last = np.random.default_rng(74).standard_normal(cfg["n_vocab"]).astype(np.float32)
        last[[17, 402]] = 9.0                                    # a tie: the first maximum wins
        g.kv_load(k, v, n_pos, logits=last)
        assert g.n_past() == n_pos

        def restored():
            o = orc.Decoder(model, n_ctx)
            ok, ov = o.caches()
            ok[:, :, :n_pos] = k
            ov[:, :, :n_pos] = v
            return o

        o = restored()
        try:
            got = g.generate([], 4)
            want, nxt, pos = [], 17, n_pos
            for _ in range(4):
                want.append(nxt)
                lg = o.forward(nxt, pos)
                pos += 1
                nxt = orc.orc().orc_argmax(orc._p(lg), cfg["n_vocab"])
            assert list(got) == want
        finally:
            o.close()

        g.kv_load(k, v, n_pos)                                   # no logits
        out = np.zeros(2, np.int32)
        assert amd.lib().sllm_gfx950_generate_greedy(g.m, g.c, None, 0, 2, amd.ptr(out)) == -1
        o = restored()
        try:
            tok = _tokens(1, cfg["n_vocab"], 75)[0]
            lg = o.forward(tok, gap)
            assert np.array_equal(bits(g.forward(tok, gap)), bits(lg)), "gapped forward"
            more = g.generate([], 2)                             # continues from the gapped forward
            first = orc.orc().orc_argmax(orc._p(lg), cfg["n_vocab"])
            second = orc.orc().orc_argmax(orc._p(o.forward(first, gap + 1)), cfg["n_vocab"])
            assert list(more) == [first, second]
        finally:
            o.close()
    finally:
        g.close()


def test_full_2b_decode_after_a_1024_position_prefix(amd, orc, dev):
    """The decode leg's workload in full: all 30 blocks at BitNet-2B shape
    with the 128256-row F16 output, over a restored 1024-position cache of
    binary16 values, two tokens at positions 1024 and 1025 -- every int32 dot,
    every activation and the logits bit for bit against the oracle."""
    cfg = dict(amd.BITNET_2B)
    n_pos = 1024
    print("[decode] building the 2B model and a 1024-position prefix", flush=True)
    model = amd.synth_model(cfg, 2)
    k, v = _kv_prefix(cfg, n_pos, 81)
    g, o = amd.DeviceDecoder(dev, model, n_pos + 4), orc.Decoder(model, n_pos + 4)
    ok, ov = o.caches()
    ok[:, :, :n_pos] = k
    ov[:, :, :n_pos] = v
    g.kv_load(k, v, n_pos)
    g.trace_start()
    try:
        for i, tok in enumerate(_tokens(2, cfg["n_vocab"], 82)):
            print(f"[decode] 2B token at {n_pos + i}", flush=True)
            _compare_step(g, o, tok, n_pos + i, "2b-prefix")
    finally:
        g.trace_stop()
        g.close()
        o.close()


def test_device_expf_matches_the_c_library(amd, dev):
    """The softmax tail's expf as the device build computes it
    (sllm_gfx950_diag_expf) against the host C library, bit for bit, on
    every 17th float bit pattern (252,645,136 inputs; NaN against NaN counts
    as equal) -- the host build of the same restatement is held against the
    library on all 2^32 in tests/test_decode_host.py."""
    stride, chunk = 17, 1 << 26
    total = (1 << 32) // stride + 1
    out = dev.alloc(4 * chunk)
    bad = 0
    try:
        for start in range(0, total, chunk):
            n = min(chunk, total - start)
            first = (start * stride) & 0xFFFFFFFF
            amd.check(amd.lib().sllm_gfx950_diag_expf(first, stride, n, out.vp), "diag_expf")
            got = out.download(np.float32, n)
            want = np.empty(n, np.float32)
            amd.synth_lib().sllm_expf_strided(first, stride, n, amd.ptr(want), 16)
            diff = (got.view(np.uint32) != want.view(np.uint32)) & ~(np.isnan(got) & np.isnan(want))
            bad += int(diff.sum())
            print(f"[expf] {start + n}/{total} inputs, {bad} differ", flush=True)
    finally:
        out.free()
    assert bad == 0

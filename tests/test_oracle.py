"""The oracle, pinned before it is trusted.

Each oracle function is checked against something other than itself:
  * upstream-captured vectors the reference's own tests hold
    (tests/golden/i2s-converter.txt, i2s-reference.txt there; extracted into
    tests/golden/*.json by tests/golden/make_fixtures.py);
  * the reference's known-answer tests (tests/test_i2s.c:431-483,
    tests/test_ops.c:77-135 there);
  * closed forms (brute-force sums, the act_sum identity);
  * the reference's own sources compiled into oracle/_ref (when built).
A few tests plant a plausible mistake in a numpy restatement and show the
same check rejects it, so the checks can fail.
"""
import json
import os
import struct

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
MAP2BIT = np.array([-1.0, 0.0, 1.0, 0.0], np.float32)      # src/quant.c:126-138


def _hexbytes(s):
    return np.frombuffer(bytes.fromhex(s), np.uint8).copy()


def _hexf32(words):
    return np.array([struct.unpack(">f", bytes.fromhex(w))[0] for w in words], np.float32)


@pytest.fixture(scope="module")
def converter():
    with open(os.path.join(GOLDEN, "i2s_converter.json")) as f:
        return json.load(f)["cases"]


@pytest.fixture(scope="module")
def gemv_records():
    with open(os.path.join(GOLDEN, "i2s_reference.json")) as f:
        return json.load(f)["gemv"]


# ---------------------------------------------------------------------------
# layout: orc_code / orc_scale / orc_dequant / orc_pack_converter
# ---------------------------------------------------------------------------

def test_upstream_converter_vectors_decode_with_the_oracle_layout(orc, converter):
    """Upstream's independent read-back (dequantize_row_i2_s) of 34 packed
    buffers: the oracle's orc_code must decode every element identically,
    and orc_scale must find the f32 scale at byte n/4."""
    checked = 0
    for case in converter:
        n = case["n"]
        want_scale = _hexf32([case["scale_f32_hex"]])[0]
        for rule in ("gguf_py", "bitnet_c"):
            packed = _hexbytes(case["rules"][rule]["packed_hex"])
            assert packed.size == n // 4 + 32 + (1 if n % 4 else 0) or packed.size == case["packed_bytes"]
            want = _hexf32(case["rules"][rule]["decoded_f32_hex"])
            got = MAP2BIT[orc.codes(packed, n)]
            np.testing.assert_array_equal(got, want, err_msg=f"n={n} rule={rule}")
            assert orc.scale(packed, n) == want_scale
            checked += n
    assert checked > 2 * 10000


def test_oracle_dequant_matches_code_times_scale(orc, converter):
    for case in converter:
        n = case["n"]
        packed = _hexbytes(case["rules"]["gguf_py"]["packed_hex"])
        s = orc.scale(packed, n)
        want = _hexf32(case["rules"]["gguf_py"]["decoded_f32_hex"]) * s
        np.testing.assert_array_equal(orc.dequant(packed, n), want)


def test_planted_layout_mistakes_fail_the_converter_vectors(converter):
    """Reversed fields (shift 2f) and a consecutive-element packing are the
    two historical misreadings (src/quant.c:85-96); both must be rejected."""
    def decode(packed, n, variant):
        out = np.empty(n, np.float32)
        for k in range(n):
            if variant == "reversed_fields":
                byte = packed[(k // 128) * 32 + k % 32]
                code = (byte >> (2 * ((k % 128) // 32))) & 3
            else:  # consecutive
                byte = packed[k // 4]
                code = (byte >> (6 - 2 * (k % 4))) & 3
            out[k] = MAP2BIT[code]
        return out

    for variant in ("reversed_fields", "consecutive"):
        bad = 0
        for case in converter:
            n = case["n"]
            if n > 1024:
                continue
            packed = _hexbytes(case["rules"]["gguf_py"]["packed_hex"])
            want = _hexf32(case["rules"]["gguf_py"]["decoded_f32_hex"])
            bad += int(np.any(decode(packed, n, variant) != want))
        assert bad > 0, variant


def test_converter_packer_reproduces_upstream_bytes_on_whole_blocks(orc, converter):
    """Packing the decoded codes by the converter's definition
    (tests/harness.h:105-126) must give back upstream's bytes for every case
    made of whole 128-element blocks, under both upstream rules."""
    n_checked = 0
    for case in converter:
        n = case["n"]
        if n % 128:
            continue
        for rule in ("gguf_py", "bitnet_c"):
            packed = _hexbytes(case["rules"][rule]["packed_hex"])
            codes = (_hexf32(case["rules"][rule]["decoded_f32_hex"]) + 1).astype(np.uint8)
            got = orc.pack_converter(codes)
            np.testing.assert_array_equal(got[: n // 4], packed[: n // 4], err_msg=f"n={n} {rule}")
            n_checked += 1
    assert n_checked == 10


def test_field_order_is_top_down_within_each_byte(orc):
    """tests/test_i2s.c:178-211: field a of every element gets code a % 3."""
    n = 1024
    codes = ((np.arange(n) // 32) % 3).astype(np.uint8)
    packed = orc.pack_converter(codes)
    np.testing.assert_array_equal(orc.codes(packed, n), codes)


def test_layout_matches_the_converter_definition_over_two_4096_blocks(orc):
    """tests/test_ops.c:77-116: codes (k*7 + k/128) % 3 over 8192 weights."""
    n = 8192
    k = np.arange(n)
    codes = ((k * 7 + k // 128) % 3).astype(np.uint8)
    packed = orc.pack_converter(codes)
    np.testing.assert_array_equal(orc.codes(packed, n), codes)


def test_scale_sits_after_the_packed_weights(orc):
    """tests/test_ops.c:118-135, including a decoy just before the scale."""
    n = 1024
    packed = np.zeros(n // 4 + 32, np.uint8)
    packed[n // 4: n // 4 + 4] = np.frombuffer(struct.pack("<f", 0.03125), np.uint8)
    packed[n // 4 - 4: n // 4] = np.frombuffer(struct.pack("<f", 99.0), np.uint8)
    assert orc.scale(packed, n) == np.float32(0.03125)


def test_row_and_dequant_differ_only_by_sign_and_scale(orc):
    """tests/test_i2s.c:213-242."""
    n = 512
    codes = (np.arange(n) % 3).astype(np.uint8)
    packed = orc.pack_converter(codes)
    packed[n // 4: n // 4 + 4] = np.frombuffer(struct.pack("<f", 0.5), np.uint8)
    np.testing.assert_array_equal(orc.dequant(packed, n),
                                  np.float32(0.5) * (codes.astype(np.float32) - 1))


# ---------------------------------------------------------------------------
# quantiser: orc_quant_act
# ---------------------------------------------------------------------------

def test_quantiser_reproduces_the_upstream_lcg_activation(orc, gemv_records):
    """The fixture pins act_scale and act_sum that the reference's quantiser
    produces on the fixed LCG activation at n=2560 and n=6912."""
    seen = set()
    for rec in gemv_records:
        n = rec["n"]
        q, s, total = orc.quant_act(orc.lcg_activation(n))
        assert s == np.float32(float(rec["act_scale"])), rec["tensor"]
        assert total == rec["act_sum"], rec["tensor"]
        assert int(q.astype(np.int64).sum()) == total
        seen.add(n)
    assert seen == {2560, 6912}


def _quant_np(x, rounding="half_away"):
    x = np.asarray(x, np.float32)
    amax = np.float32(np.max(np.abs(x)))
    s = np.float32(127.0) / amax if amax > 0 else np.float32(0)
    xs = x * s
    if rounding == "half_away":
        r = np.sign(xs) * np.floor(np.abs(xs) + np.float32(0.5))
    else:
        r = np.rint(xs)
    q = np.clip(r, -128, 127).astype(np.int32)
    return q, (np.float32(127.0) / amax), int(q.sum())


def test_numpy_restatement_agrees_then_planted_quantiser_mistakes_fail(orc, gemv_records):
    rec = [r for r in gemv_records if r["n"] == 2560][0]
    x = orc.lcg_activation(2560)
    q_ok, _, sum_ok = _quant_np(x)
    q_c, _, sum_c = orc.quant_act(x)
    np.testing.assert_array_equal(q_ok, q_c.astype(np.int32))
    assert sum_ok == rec["act_sum"]
    # banker's rounding differs from roundf on ties
    ties = np.array([0.5, 1.5, 2.5, 4.5, -0.5, 127.0] * 8, np.float32)
    assert _quant_np(ties, rounding="rint")[2] != orc.quant_act(ties)[2]
    assert np.any(_quant_np(ties, rounding="rint")[0] != orc.quant_act(ties)[0])
    # truncating instead of rounding, and max(x) instead of max|x|, both
    # miss the fixture's act_sum at n=2560
    xs = x * (np.float32(127.0) / np.float32(np.max(np.abs(x))))
    assert int(np.clip(np.trunc(xs), -128, 127).astype(np.int64).sum()) != rec["act_sum"]
    s_bad = np.float32(127.0) / np.float32(np.max(x))
    r_bad = np.sign(x * s_bad) * np.floor(np.abs(x * s_bad) + np.float32(0.5))
    assert (s_bad != np.float32(float(rec["act_scale"])) or
            int(np.clip(r_bad, -128, 127).astype(np.int64).sum()) != rec["act_sum"])


def test_activation_quantiser_matches_the_reference_rules(orc):
    """tests/test_i2s.c:458-483: zero row -> scale 0; max 2 -> scale 63.5."""
    q, s, total = orc.quant_act(np.zeros(256, np.float32))
    assert s == 0.0 and total == 0 and not q.any()
    u = np.where(np.arange(256) % 3 == 0, 2.0, -1.0).astype(np.float32)
    q, s, total = orc.quant_act(u)
    assert s == np.float32(63.5)
    np.testing.assert_array_equal(q, np.where(np.arange(256) % 3 == 0, 127, -64).astype(np.int8))
    assert total == int(q.astype(np.int64).sum())


def test_quantiser_edge_cases(orc):
    # a single non-zero element takes the full range; negative max too
    x = np.zeros(128, np.float32)
    x[7] = -3.0
    q, s, total = orc.quant_act(x)
    assert q[7] == -127 and total == -127 and s == np.float32(127.0) / np.float32(3.0)
    # NaN is skipped by the max (a > amax is false)
    x = np.ones(128, np.float32)
    x[3] = np.nan
    _, s, _ = orc.quant_act(x)
    assert s == np.float32(127.0)


# ---------------------------------------------------------------------------
# dot products: closed form and agreement of the three oracle kernels
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("n", [128, 256, 640, 2560, 6912])
def test_dot_kernels_equal_the_brute_force_sum(orc, n):
    rng = np.random.default_rng(n)
    for _ in range(4):
        codes = rng.integers(0, 3, n, dtype=np.uint8)
        q = rng.integers(-128, 128, n, dtype=np.int8)
        packed = orc.pack_converter(codes)
        want = int((codes.astype(np.int64) * q.astype(np.int64)).sum())
        ternary = int(((codes.astype(np.int64) - 1) * q.astype(np.int64)).sum())
        assert want - int(q.astype(np.int64).sum()) == ternary     # docs/BITNET-LIFECYCLE.md:52
        for path in (orc.DOT_SCALAR, orc.DOT_V3, orc.DOT_VNNI):
            assert orc.dot(packed, q, n, path) == want


def test_dot_extremes_do_not_saturate(orc):
    """All codes 2 against all -128 / +127: the int16 stage of maddubs stays
    exact (src/i2s_gemm.c:169-175)."""
    n = 6912
    packed = orc.pack_converter(np.full(n, 2, np.uint8))
    for v in (-128, 127):
        q = np.full(n, v, np.int8)
        for path in (orc.DOT_SCALAR, orc.DOT_V3, orc.DOT_VNNI):
            assert orc.dot(packed, q, n, path) == 2 * v * n


def test_gemv_rows_and_parallel_gemv_agree(orc):
    rng = np.random.default_rng(7)
    n_rows, n = 1536, 2560
    codes = rng.integers(0, 3, (n_rows, n), dtype=np.uint8)
    packed = np.concatenate([orc.pack_converter(r)[: n // 4] for r in codes] + [np.zeros(32, np.uint8)])
    q = rng.integers(-128, 128, n, dtype=np.int8)
    want = (codes.astype(np.int64) @ q.astype(np.int64)).astype(np.int32)
    np.testing.assert_array_equal(orc.gemv(packed, n_rows, n, q, orc.DOT_V3), want)
    pool = orc.Pool(3)
    out = np.empty(n_rows, np.int32)
    pool.gemv(packed, n_rows, n, q, out, orc.DOT_VNNI)
    pool.close()
    np.testing.assert_array_equal(out, want)


# ---------------------------------------------------------------------------
# epilogue: orc_epilogue
# ---------------------------------------------------------------------------

def test_epilogue_reproduces_upstream_values(orc, gemv_records):
    """Each record holds upstream's raw dots and epilogue outputs for the same
    rows: (dot - act_sum) * (w_scale / act_scale) must print identically."""
    for rec in gemv_records:
        s = np.float32(float(rec["act_scale"]))
        ws = np.float32(float(rec["w_scale"]))
        for d, want in zip(rec["values"], rec["epilogue_values"]):
            assert f"{float(orc.epilogue(d, rec['act_sum'], s, ws)):.6f}" == want, rec["tensor"]
        # the vectorised restatement agrees with the C oracle bit for bit
        got = orc.epilogue_np(rec["values"], rec["act_sum"], s, ws)
        np.testing.assert_array_equal(got, orc.epilogue_rows(rec["values"], rec["act_sum"], s, ws))


def test_planted_epilogue_mistake_fails_upstream_values(gemv_records):
    """Dropping the act_sum term (the 'suspicious' reading) is rejected."""
    rec = gemv_records[0]
    s = np.float32(float(rec["act_scale"]))
    ws = np.float32(float(rec["w_scale"]))
    post = ws / s
    got = [f"{float(np.float32(d) * post):.6f}" for d in rec["values"][:8]]
    assert got != rec["epilogue_values"]


def test_epilogue_is_reproduced_verbatim(orc):
    """tests/test_i2s.c:431-456."""
    dots = [0, 1, -1, 1000, -1000, 123456, -123456]
    sums = [0, 5, -5, 0, 0, 77, -77]
    scales = np.array([1.0, 2.0, 0.5, 127.0, 0.007874, 42.0, 3.5], np.float32)
    w = np.array([1.0, -1.0, 0.25, 2.16316128, 1.21885478, 2.17397785, 0.5], np.float32)
    for d, a, s, ws in zip(dots, sums, scales, w):
        want = np.float32(d - a) * (ws / s)
        assert orc.epilogue(d, a, s, ws).tobytes() == np.float32(want).tobytes()
    assert orc.epilogue(1000, 100, 1.0, 1.0) == 900.0
    assert orc.epilogue(1000, 0, 1.0, 1.0) == 1000.0


def test_zero_row_epilogue_is_nan(orc):
    """A zero activation row has scale 0, so post = inf and 0*inf = NaN
    (tests/test_i2s.c:458-469)."""
    assert np.isnan(orc.epilogue(0, 0, 0.0, 1.5))


# ---------------------------------------------------------------------------
# the reference's own sources (oracle/_ref), when built
# ---------------------------------------------------------------------------

needs_ref = pytest.mark.skipif(
    not os.path.exists(os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                                    "oracle", "_ref", "libsllm_ref.so")),
    reason="oracle/_ref not built (reference tree absent at build time)")


@needs_ref
def test_restatement_matches_the_compiled_reference(orc):
    import ctypes
    r = orc.ref()
    rng = np.random.default_rng(11)
    for n in (128, 384, 2560, 6912):
        for trial in range(3):
            x = rng.standard_normal(n).astype(np.float32) * np.float32(rng.uniform(0.01, 50))
            q_o, s_o, sum_o = orc.quant_act(x)
            q_r = np.empty(n, np.int8)
            a = orc.Act()
            r.sllm_i2s_quant_act(x.ctypes.data_as(ctypes.c_void_p), n,
                                 q_r.ctypes.data_as(ctypes.c_void_p), ctypes.byref(a))
            np.testing.assert_array_equal(q_o, q_r)
            assert (s_o, sum_o) == (np.float32(a.scale), a.sum)
            codes = rng.integers(0, 3, n, dtype=np.uint8)
            packed = orc.pack_converter(codes)
            pw = packed.ctypes.data_as(ctypes.c_void_p)
            pq = q_o.ctypes.data_as(ctypes.c_void_p)
            want = orc.dot(packed, q_o, n, orc.DOT_SCALAR)
            assert r.sllm_i2s_dot_scalar(pw, pq, n) == want
            for level in (0, 1):            # SLLM_ISA_V3, SLLM_ISA_VNNI
                r.sllm_i2s_select_level(level)
                assert r.sllm_i2s_dot(pw, pq, n) == want
            for k in range(0, n, 37):
                assert r.sllm_i2s_code(pw, k) == codes[k]
            d = int(rng.integers(-300000, 300000))
            e_r = r.sllm_i2s_epilogue(d, sum_o, float(s_o), 1.7)
            assert np.float32(e_r).tobytes() == orc.epilogue(d, sum_o, s_o, np.float32(1.7)).tobytes()
    # edge rows: zero, denormal amax (127/amax overflows to inf), huge values,
    # a NaN element, a ramp full of ties after scaling
    n = 256
    for x in (np.zeros(n, np.float32), np.full(n, 1e-40, np.float32),
              np.where(np.arange(n) % 2 == 0, 3e38, -3e38).astype(np.float32),
              np.where(np.arange(n) == 5, np.nan, 1.0).astype(np.float32),
              np.linspace(-0.5, 0.5, n).astype(np.float32)):
        q_o, s_o, sum_o = orc.quant_act(x)
        q_r = np.empty(n, np.int8)
        a = orc.Act()
        r.sllm_i2s_quant_act(x.ctypes.data_as(ctypes.c_void_p), n, q_r.ctypes.data_as(ctypes.c_void_p), ctypes.byref(a))
        np.testing.assert_array_equal(q_o, q_r)
        assert np.float32(a.scale).tobytes() == s_o.tobytes() and a.sum == sum_o
    # the LCG golden through the reference's quantiser too
    x = orc.lcg_activation(2560)
    q_r = np.empty(2560, np.int8)
    a = orc.Act()
    r.sllm_i2s_quant_act(x.ctypes.data_as(ctypes.c_void_p), 2560, q_r.ctypes.data_as(ctypes.c_void_p), ctypes.byref(a))
    assert np.float32(a.scale) == np.float32(42.3747139) and a.sum == 6643

"""GGUF v3 images read by sllm_gfx950_gguf_describe (the host half of
sllm_gfx950_model_load_gguf) against the reference's own reader.

Every image is accepted or refused with the status the reference returns for
it: each case states that status (from the reference's rules,
src/gguf.c:488-700 for the container and src/forward.c:269-455 for the
model), and where oracle/_ref is built the reference's
sllm_gguf_open_memory + sllm_model_load is run on the same bytes and must
agree. An accepted image must hand back the model's hyper-parameters and,
for every tensor, the offset in the image of exactly the bytes the writer put
there. No device is needed.
"""
import struct

import numpy as np
import pytest

from oracle import gguf_synth

TINY = dict(n_layer=2, n_embd=256, n_ff=512, n_head=4, n_head_kv=2, n_rot=64, n_vocab=300,
            eps=1e-5, rope_base=500000.0)
ARCH = "bitnet-b1.58"
VT_U8, VT_I8, VT_U16, VT_I16, VT_U32, VT_I32, VT_F32, VT_BOOL, VT_STR, VT_ARR, VT_U64 = range(11)
T_F32, T_F16, T_Q8_0, T_I2S, T_I8S = 0, 1, 8, 36, 37


def s8(b):
    if isinstance(b, str):
        b = b.encode()
    return struct.pack("<Q", len(b)) + b


def kv_raw(key, vtype, payload):
    return s8(key) + struct.pack("<I", vtype) + payload


def kv_u32(key, v):
    return kv_raw(key, VT_U32, struct.pack("<I", v))


def kv_f32(key, v):
    return kv_raw(key, VT_F32, struct.pack("<f", v))


def kv_str(key, v):
    return kv_raw(key, VT_STR, s8(v))


def kv_arr(key, etype, n, payload):
    return kv_raw(key, VT_ARR, struct.pack("<IQ", etype, n) + payload)


class Parts:
    """A GGUF image as editable pieces: metadata entries (bytes, keyed by name
    for replacement), tensor table entries and their data."""

    def __init__(self, model):
        cfg = model["cfg"]
        e, f = cfg["n_embd"], cfg["n_ff"]
        gqa = e // cfg["n_head"] * cfg["n_head_kv"]
        self.kvs = [("general.architecture", kv_str("general.architecture", ARCH))]
        for key, name in [("block_count", "n_layer"), ("embedding_length", "n_embd"),
                          ("feed_forward_length", "n_ff"), ("attention.head_count", "n_head"),
                          ("attention.head_count_kv", "n_head_kv"), ("rope.dimension_count", "n_rot")]:
            self.kvs.append((key, kv_u32(f"{ARCH}.{key}", cfg[name])))
        self.kvs.append(("context_length", kv_u32(f"{ARCH}.context_length", 4096)))
        self.kvs.append(("vocab_size", kv_u32(f"{ARCH}.vocab_size", cfg["n_vocab"])))
        self.kvs.append(("eps", kv_f32(f"{ARCH}.attention.layer_norm_rms_epsilon", cfg["eps"])))
        self.kvs.append(("freq_base", kv_f32(f"{ARCH}.rope.freq_base", cfg["rope_base"])))
        # [name(bytes), dims, type, data bytes, key for the describe map]
        self.tensors = [[b"token_embd.weight", (e, cfg["n_vocab"]), T_F16, model["tok_embd"].tobytes(), "tok_embd"],
                        [b"output_norm.weight", (e,), T_F32, model["output_norm"].tobytes(), "output_norm"]]
        dims = {"wq": (e, e), "wk": (e, gqa), "wv": (e, gqa), "wo": (e, e), "w_gate": (e, f), "w_up": (e, f),
                "w_down": (f, e), "attn_norm": (e,), "attn_sub_norm": (e,), "ffn_norm": (e,),
                "ffn_sub_norm": (f,)}
        for il, layer in enumerate(model["layers"]):
            for key, arr in layer.items():
                ttype = T_I2S if key.startswith("w") else T_F32
                name = f"blk.{il}.{gguf_synth._NAMES[key]}.weight".encode()
                self.tensors.append([name, dims[key], ttype, np.ascontiguousarray(arr).tobytes(), (il, key)])
        self.align = 32
        self.offsets = None        # tensor index -> offset override

    def kv(self, name, entry):
        """Replace (entry bytes) or drop (None) the metadata entry `name`."""
        i = [k for k, _ in self.kvs].index(name)
        if entry is None:
            del self.kvs[i]
        else:
            self.kvs[i] = (name, entry)
        return self

    def tensor(self, key):
        return next(t for t in self.tensors if t[4] == key)

    @staticmethod
    def nbytes(dims, ttype):
        n = int(np.prod(dims, dtype=object))
        size = {T_F32: 4 * n, T_F16: 2 * n, T_I2S: n // 4 + 32, T_Q8_0: n // 32 * 34}.get(ttype)
        return size if size is not None and n < 1 << 26 else 0

    def build(self, magic=b"GGUF", version=3, n_t=None, n_kv=None):
        """The image; data shorter than its tensor's declared size is padded
        with zeros so that a reshaped tensor never runs into its neighbour.
        Sets kv_end / table_end (byte positions) and data_at / tensor_at."""
        table, blobs, offsets, at = [], [], [], 0
        for t in self.tensors:
            name, dims, ttype, data = t[:4]
            data = data + b"\0" * max(0, self.nbytes(dims, ttype) - len(data))
            pad = (-len(data)) % self.align
            offsets.append(at)
            blobs.append(data + b"\0" * pad)
            at += len(data) + pad
        if self.offsets:
            for i, o in self.offsets.items():
                offsets[i] = o
        for t, off in zip(self.tensors, offsets):
            name, dims, ttype = t[:3]
            table.append(s8(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
                         + struct.pack("<IQ", ttype, off))
        n_t = len(self.tensors) if n_t is None else n_t
        n_kv = len(self.kvs) if n_kv is None else n_kv
        head = magic + struct.pack("<IQQ", version, n_t, n_kv) + b"".join(e for _, e in self.kvs)
        meta = head + b"".join(table)
        self.kv_end, self.table_end = len(head), len(meta)
        data_at = len(meta) + (-len(meta)) % self.align
        self.data_at, self.tensor_at = data_at, offsets
        return meta + b"\0" * (data_at - len(meta)) + b"".join(blobs)


@pytest.fixture(scope="module")
def model(amd):
    return amd.synth_model(TINY, 21)


def ref_status(orc, image):
    if not orc.ref_available():
        return None
    import ctypes
    buf = np.frombuffer(image, np.uint8) if len(image) else np.zeros(1, np.uint8)
    st = ctypes.c_int(0)
    r = orc.ref().ref_model_open(buf.ctypes.data_as(ctypes.c_void_p), len(image), ctypes.byref(st))
    if r:
        orc.ref().ref_model_close(r)
    return st.value


def check_status(amd, orc, image, want):
    got = amd.gguf_describe(image)[0]
    ref = ref_status(orc, image)
    assert got == want, f"describe gave {got}, the reference's rule says {want}"
    if ref is not None:
        assert ref == want, f"the reference's loader gave {ref}, expected {want}"


def test_a_valid_image_describes_the_model_in_place(amd, orc, model):
    p = Parts(model)
    image = p.build()
    st, cfg, tensors = amd.gguf_describe(image)
    assert st == 0 and (ref_status(orc, image) in (None, 0))
    for k, v in TINY.items():
        assert np.float32(cfg[k]) == np.float32(v), k
    for i, t in enumerate(p.tensors):
        at = tensors[t[4]]
        assert at == p.data_at + p.tensor_at[i], t[0]
        assert image[at:at + len(t[3])] == t[3], t[0]


def test_the_synthetic_writer_image_is_read_the_same(amd, model):
    """The image the decode tests hand the reference (oracle/gguf_synth.py)."""
    image = gguf_synth.gguf_image(model)
    st, cfg, tensors = amd.gguf_describe(image)
    assert st == 0 and cfg["n_layer"] == TINY["n_layer"] and cfg["n_vocab"] == TINY["n_vocab"]
    w = model["layers"][1]["w_down"]
    assert image[tensors[(1, "w_down")]:tensors[(1, "w_down")] + w.nbytes] == w.tobytes()


def test_alignment_key_moves_the_data(amd, orc, model):
    p = Parts(model)
    p.kvs.append(("align", kv_u32("general.alignment", 256)))
    p.align = 256
    image = p.build()
    st, _, tensors = amd.gguf_describe(image)
    assert st == 0 and p.data_at % 256 == 0 and ref_status(orc, image) in (None, 0)
    assert tensors["tok_embd"] == p.data_at


def _container_cases(model):
    """(id, image bytes, status) for the container's rules."""
    P = lambda: Parts(model)  # noqa: E731
    good = P().build()
    cases = [
        ("empty", b"", -12),
        ("three_bytes", b"GGU", -12),
        ("bad_magic", b"GGUX" + good[4:], -10),
        ("version_2", P().build(version=2), -11),
        ("header_cut", good[:20], -12),
        ("too_many_tensors", P().build(n_t=(1 << 20) + 1), -36),
        ("too_many_kv", P().build(n_kv=(1 << 22) + 1), -36),
    ]
    # counts that the file cannot hold: the image ends right after the last
    # real entry, so the next read runs off the end
    p = P()
    image = p.build(n_kv=1 << 22)
    cases.append(("kv_count_past_file", image[:p.kv_end], -12))
    p = P()
    image = p.build(n_t=1 << 20)
    cases.append(("tensor_count_past_file", image[:p.table_end], -12))
    p = P()
    p.build()
    cases.append(("cut_in_metadata", good[:100], -12))
    cases.append(("cut_in_tensor_table", good[:(p.kv_end + p.table_end) // 2], -12))
    p = P()
    p.kvs.insert(1, ("x", kv_raw("x.unknown", 13, b"")))
    cases.append(("value_type_13", p.build(), -14))
    p = P()
    p.kvs.insert(1, ("x", kv_arr("x.nested", VT_ARR, 1, b"")))
    cases.append(("array_of_arrays", p.build(), -14))
    p = P()
    p.kvs.insert(1, ("x", kv_arr("x.badelem", 13, 1, b"")))
    cases.append(("array_elem_type_13", p.build(), -14))
    p = P()
    p.kvs.insert(1, ("x", kv_arr("x.huge", VT_U8, (1 << 28) + 1, b"")))
    cases.append(("array_too_long", p.build(), -36))
    p = P()
    p.kvs.insert(1, ("x", kv_arr("x.strs", VT_STR, 1 << 27, b"")))
    cases.append(("string_array_past_file", p.build(), -36))
    p = P()
    p.kvs.insert(1, ("x", kv_arr("x.cut", VT_U32, 1 << 26, b"")))
    cases.append(("u32_array_past_file", p.build(), -12))
    p = P()
    p.kvs.insert(1, ("x", kv_raw("x.longstr", VT_STR, struct.pack("<Q", (1 << 30) + 1))))
    cases.append(("string_over_limit", p.build(), -12))
    p = P()
    p.kvs.insert(1, ("x", kv_u32("general.architecture", 7)))
    cases.append(("duplicate_key", p.build(), -18))
    p = P()
    p.kvs.insert(1, ("x", kv_u32("general.architecture", 7)))
    p.kvs.insert(2, ("y", kv_raw("x.unknown", 13, b"")))
    cases.append(("duplicate_reported_before_later_error", p.build(), -18))
    p = P()
    p.kvs.insert(1, ("y", kv_raw("x.unknown", 13, b"")))
    p.kvs.insert(2, ("x", kv_u32("general.architecture", 7)))
    cases.append(("earlier_error_reported_before_duplicate", p.build(), -14))
    p = P()
    p.kvs.insert(1, ("x", kv_u32(b"general.architecture\0tail", 7)))
    cases.append(("duplicate_up_to_embedded_nul", p.build(), -18))
    for n_dims, id_ in ((0, "rank_0"), (5, "rank_5")):
        p = P()
        t = p.tensor("output_norm")
        image = p.build()
        name = s8(t[0])
        at = image.index(name) + len(name)
        image = image[:at] + struct.pack("<I", n_dims) + image[at + 4:]
        cases.append((id_, image, -15))
    p = P()
    p.tensor("output_norm")[1] = (0,)
    cases.append(("zero_dim", p.build(), -15))
    p = P()
    p.tensors.append([b"x.overflow", (1 << 32, 1 << 32), T_F32, b"", "x"])
    cases.append(("dim_product_overflow", p.build(), -15))
    for ttype in (4, 43, 1000):
        p = P()
        p.tensors.append([b"x.badtype", (32,), ttype, b"\0" * 32, "x"])
        cases.append((f"tensor_type_{ttype}", p.build(), -15))
    p = P()
    p.kvs.append(("align", kv_u32("general.alignment", 48)))
    cases.append(("alignment_48", p.build(), -16))
    p = P()
    p.kvs.append(("align", kv_u32("general.alignment", 0)))
    cases.append(("alignment_0", p.build(), -16))
    p = P()
    p.kvs.append(("align", kv_raw("general.alignment", VT_U64, struct.pack("<Q", 48))))
    cases.append(("alignment_not_u32_is_ignored", p.build(), 0))
    p = P()
    p.tensors = []
    p.kvs.append(("align", kv_u32("general.alignment", 1 << 20)))
    cases.append(("data_start_past_file", p.build(), -12))
    p = P()
    p.offsets = {1: len(good)}
    cases.append(("extent_past_blob", p.build(), -17))
    p = P()
    p.offsets = {len(p.tensors) - 1: 0}
    cases.append(("overlapping_extents", p.build(), -17))
    p = P()
    p.tensors.append([b"x.unsized_i8s", (64,), T_I8S, b"", "x"])
    p.offsets = {len(p.tensors) - 1: 1 << 40}
    cases.append(("unsized_type_extent_not_checked", p.build(), 0))
    p = P()
    p.tensors.append([b"x.ragged_i2s", (6,), T_I2S, b"", "x"])
    p.offsets = {len(p.tensors) - 1: 1 << 40}
    cases.append(("i2s_not_whole_bytes_not_placed", p.build(), 0))
    p = P()
    p.tensors.append([b"x.ragged_q8", (33,), T_Q8_0, b"", "x"])
    p.offsets = {len(p.tensors) - 1: 1 << 40}
    cases.append(("q8_not_whole_blocks_not_placed", p.build(), 0))
    return cases


def _model_cases(model):
    """(id, image bytes, status) for the model's rules."""
    P = lambda: Parts(model)  # noqa: E731
    cases = [
        ("no_architecture", P().kv("general.architecture", None).build(), -30),
        ("other_architecture", P().kv("general.architecture", kv_str("general.architecture", "llama")).build(), -30),
        ("architecture_as_u32", P().kv("general.architecture", kv_u32("general.architecture", 1)).build(), -30),
        ("architecture_up_to_nul", P().kv("general.architecture",
                                          kv_str("general.architecture", ARCH.encode() + b"\0x")).build(), 0),
        ("no_block_count", P().kv("block_count", None).build(), -31),
        ("block_count_i32", P().kv("block_count", kv_raw(f"{ARCH}.block_count", VT_I32,
                                                         struct.pack("<i", 2))).build(), -31),
        ("block_count_u32_array", P().kv("block_count", kv_arr(f"{ARCH}.block_count", VT_U32, 2,
                                                               struct.pack("<II", 2, 9))).build(), 0),
        ("block_count_empty_array", P().kv("block_count", kv_arr(f"{ARCH}.block_count", VT_U32, 0, b"")).build(),
         -31),
        ("no_context_length", P().kv("context_length", None).build(), -31),
        ("no_eps", P().kv("eps", None).build(), -31),
        ("eps_f32_array", P().kv("eps", kv_arr(f"{ARCH}.attention.layer_norm_rms_epsilon", VT_F32, 1,
                                               struct.pack("<f", 1e-5))).build(), 0),
        ("freq_base_u32", P().kv("freq_base", kv_u32(f"{ARCH}.rope.freq_base", 10000)).build(), -31),
        ("zero_layers", P().kv("block_count", kv_u32(f"{ARCH}.block_count", 0)).build(), -34),
        ("65_layers", P().kv("block_count", kv_u32(f"{ARCH}.block_count", 65)).build(), -34),
        ("negative_width", P().kv("embedding_length", kv_u32(f"{ARCH}.embedding_length", 1 << 31)).build(), -34),
        ("heads_not_multiple_of_kv_heads", P().kv("attention.head_count_kv",
                                                  kv_u32(f"{ARCH}.attention.head_count_kv", 3)).build(), -34),
        ("width_not_multiple_of_heads", P().kv("attention.head_count",
                                               kv_u32(f"{ARCH}.attention.head_count", 6)).build(), -34),
        ("rot_above_head_dim", P().kv("rope.dimension_count",
                                      kv_u32(f"{ARCH}.rope.dimension_count", 65)).build(), -34),
        ("more_layers_than_tensors", P().kv("block_count", kv_u32(f"{ARCH}.block_count", 3)).build(), -34),
    ]
    p = P()
    p.tensors = [t for t in p.tensors if t[4] != (1, "wv")]
    cases.append(("missing_tensor", p.build(), -34))
    p = P()
    t = p.tensor("tok_embd")
    t[2], t[3] = T_F32, t[3] + t[3]
    cases.append(("embedding_f32", p.build(), -34))
    p = P()
    p.tensor((0, "attn_norm"))[1] = (TINY["n_embd"], 1)
    cases.append(("norm_of_rank_2", p.build(), -34))
    p = P()
    p.tensor((0, "ffn_sub_norm"))[1] = (TINY["n_embd"],)
    cases.append(("ffn_sub_norm_of_width_n_embd", p.build(), -34))
    p = P()
    p.tensor((1, "wk"))[1] = (TINY["n_embd"], TINY["n_embd"])
    cases.append(("k_projection_of_n_embd_rows", p.build(), -34))
    p = P()
    t = p.tensor((0, "w_down"))
    t[1] = (TINY["n_ff"] - 64, TINY["n_embd"])
    cases.append(("i2s_width_not_whole_blocks", p.build(), -34))
    p = P()
    p.tensor((0, "wq"))[2] = T_F16
    cases.append(("projection_f16", p.build(), -34))
    p = P()
    p.tensor("output_norm")[0] = b"output_norm.weight\0x"
    cases.append(("tensor_name_up_to_nul", p.build(), 0))
    return cases


@pytest.fixture(scope="module")
def cases(model):
    return {c[0]: c[1:] for c in _container_cases(model) + _model_cases(model)}


CONTAINER = ["empty", "three_bytes", "bad_magic", "version_2", "header_cut", "too_many_tensors", "too_many_kv",
             "kv_count_past_file", "tensor_count_past_file", "cut_in_metadata", "cut_in_tensor_table",
             "value_type_13", "array_of_arrays", "array_elem_type_13", "array_too_long", "string_array_past_file",
             "u32_array_past_file", "string_over_limit", "duplicate_key", "duplicate_reported_before_later_error",
             "earlier_error_reported_before_duplicate", "duplicate_up_to_embedded_nul", "rank_0", "rank_5",
             "zero_dim", "dim_product_overflow", "tensor_type_4", "tensor_type_43", "tensor_type_1000",
             "alignment_48", "alignment_0", "alignment_not_u32_is_ignored", "data_start_past_file",
             "extent_past_blob", "overlapping_extents", "unsized_type_extent_not_checked",
             "i2s_not_whole_bytes_not_placed", "q8_not_whole_blocks_not_placed"]
MODEL = ["no_architecture", "other_architecture", "architecture_as_u32", "architecture_up_to_nul",
         "no_block_count", "block_count_i32", "block_count_u32_array", "block_count_empty_array",
         "no_context_length", "no_eps", "eps_f32_array", "freq_base_u32", "zero_layers", "65_layers",
         "negative_width", "heads_not_multiple_of_kv_heads", "width_not_multiple_of_heads", "rot_above_head_dim",
         "more_layers_than_tensors", "missing_tensor", "embedding_f32", "norm_of_rank_2",
         "ffn_sub_norm_of_width_n_embd", "k_projection_of_n_embd_rows", "i2s_width_not_whole_blocks",
         "projection_f16", "tensor_name_up_to_nul"]


def test_every_case_is_listed(cases):
    assert sorted(cases) == sorted(CONTAINER + MODEL)


@pytest.mark.parametrize("case", CONTAINER)
def test_container_rules_match_the_reference(amd, orc, cases, case):
    image, want = cases[case]
    check_status(amd, orc, image, want)


@pytest.mark.parametrize("case", MODEL)
def test_model_rules_match_the_reference(amd, orc, cases, case):
    image, want = cases[case]
    check_status(amd, orc, image, want)


def test_load_refuses_without_a_device_or_arguments(amd, model):
    import ctypes
    L = amd.lib()
    image = np.frombuffer(Parts(model).build(), np.uint8)
    m = ctypes.c_void_p()
    assert L.sllm_gfx950_model_load_gguf(image.ctypes.data_as(ctypes.c_void_p), image.size, None) == -1
    assert L.sllm_gfx950_gguf_describe(None, 0, None, None) == -1
    if not L.sllm_gfx950_is_open():
        assert L.sllm_gfx950_model_load_gguf(image.ctypes.data_as(ctypes.c_void_p), image.size,
                                             ctypes.byref(m)) == -60
    assert L.sllm_gfx950_model_load_gguf_file(b"/nonexistent/model.gguf", ctypes.byref(m)) == -3


def test_file_loader_reads_a_file_like_the_image(amd, model, tmp_path):
    import ctypes
    L = amd.lib()
    path = tmp_path / "empty.gguf"
    path.write_bytes(b"")
    m = ctypes.c_void_p()
    assert L.sllm_gfx950_model_load_gguf_file(str(path).encode(), ctypes.byref(m)) == -12
    assert L.sllm_gfx950_model_load_gguf_file(str(tmp_path).encode(), ctypes.byref(m)) == -3
    path.write_bytes(b"GGUX" + b"\0" * 64)
    assert L.sllm_gfx950_model_load_gguf_file(str(path).encode(), ctypes.byref(m)) == -10

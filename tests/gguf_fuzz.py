"""Mutation fuzz of sllm_gfx950_gguf_describe, the library's GGUF reader (the
counterpart of the reference's src/gguf.c:488-700 and the model checks of
src/forward.c:269-455), for the sanitizer run (tests/test_sanitizers.py).

Seeds: the accepted image and every refused image of tests/test_gguf_load.py
(its two-block model). Each mutant (bit flips, bytes and words set to edge values, cuts,
insertions, deletions, splices of two seeds -- mostly inside the header) is
copied into a buffer of exactly its size from the C allocator, so that a read
past the image meets a sanitizer redzone, and read. A sanitizer report ends
the process. A status outside the reader's set, or an accepted image whose
tensor data would lie outside it, is a finding: it is printed with the
mutant's bytes (hex) and the run stops with status 1.

    python tests/gguf_fuzz.py LIBRARY SECONDS SEED
"""
import ctypes
import os
import random
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
sys.path.insert(0, ROOT)
sys.path.insert(0, HERE)

STATUSES = {0, -1, -2, -10, -11, -12, -14, -15, -16, -17, -18, -30, -31, -34, -36}
EDGE_BYTES = (0x00, 0x01, 0x7F, 0x80, 0xFF, 0x03, 0x24, 0x25)
EDGE_WORDS = (0, 1, 2, 3, 31, 32, 127, 128, 255, 256, 0x7FFFFFFF, 0x80000000, 0xFFFFFFFF,
              (1 << 20) + 1, (1 << 22) + 1, 1 << 32, (1 << 63) - 1, 1 << 63, (1 << 64) - 1)


def seeds(amd):
    import test_gguf_load as t
    model = amd.synth_model(t.TINY, 11)
    good = t.Parts(model).build()
    images = [good] + [c[1] for c in t._container_cases(model) + t._model_cases(model)]
    return [bytes(i) for i in images], model["cfg"]


def extents(cfg, tensors):
    """(offset, size) of every tensor of an accepted image."""
    e, f, v = cfg["n_embd"], cfg["n_ff"], cfg["n_vocab"]
    g = e // cfg["n_head"] * cfg["n_head_kv"]
    i2s = lambda rows, k: rows * k // 4 + 32  # noqa: E731
    sizes = {"wq": i2s(e, e), "wk": i2s(g, e), "wv": i2s(g, e), "wo": i2s(e, e), "w_gate": i2s(f, e),
             "w_up": i2s(f, e), "w_down": i2s(e, f), "attn_norm": 4 * e, "attn_sub_norm": 4 * e,
             "ffn_norm": 4 * e, "ffn_sub_norm": 4 * f}
    out = [(tensors["tok_embd"], 2 * e * v), (tensors["output_norm"], 4 * e)]
    for key, off in tensors.items():
        if isinstance(key, tuple):
            out.append((off, sizes[key[1]]))
    return out


def mutate(rng, img, pool):
    b = bytearray(img)
    for _ in range(rng.randint(1, 4)):
        op = rng.randrange(8)
        span = min(len(b), 1024) if rng.random() < 0.9 else len(b)      # mostly inside the header
        at = rng.randrange(span) if span else 0
        if op == 0 and b:                                     # bit flip
            b[at] ^= 1 << rng.randrange(8)
        elif op == 1 and b:                                   # edge byte
            b[at] = rng.choice(EDGE_BYTES)
        elif op == 2 and len(b) >= 8:                         # edge word, little-endian 4 or 8 bytes
            w = rng.choice((4, 8))
            at = min(at, len(b) - w)
            b[at:at + w] = (rng.choice(EDGE_WORDS) & ((1 << (8 * w)) - 1)).to_bytes(w, "little")
        elif op == 3 and b:                                   # cut
            del b[rng.randrange(len(b) + 1):]
        elif op == 4:                                         # insert
            b[at:at] = bytes(rng.randrange(256) for _ in range(rng.randint(1, 16)))
        elif op == 5 and b:                                   # delete
            del b[at:at + rng.randint(1, 16)]
        elif op == 6 and b:                                   # small arithmetic
            b[at] = (b[at] + rng.choice((-2, -1, 1, 2))) & 0xFF
        else:                                                 # splice with another seed
            other = rng.choice(pool)
            cut = rng.randrange(len(other) + 1)
            b = b[:min(at, len(b))] + bytearray(other[cut:])
    return bytes(b)


def main():
    lib_path, seconds, seed = sys.argv[1], float(sys.argv[2]), int(sys.argv[3])
    import conftest
    amd = conftest.load_package()
    amd.LIB_PATH = lib_path
    L = amd.lib()
    libc = ctypes.CDLL(None)
    libc.malloc.restype, libc.malloc.argtypes = ctypes.c_void_p, [ctypes.c_size_t]
    libc.free.argtypes = [ctypes.c_void_p]
    pool, cfg0 = seeds(amd)
    rng = random.Random(seed)
    hist, n, t_end = {}, 0, time.monotonic() + seconds
    d = amd.ModelDesc()
    layers = (amd.LayerDesc * amd.GGUF_MAX_LAYERS)()
    while time.monotonic() < t_end:
        img = mutate(rng, rng.choice(pool), pool)
        buf = libc.malloc(max(len(img), 1))
        ctypes.memmove(buf, img, len(img))
        st = L.sllm_gfx950_gguf_describe(buf, len(img), ctypes.byref(d), layers)
        bad = None
        if st not in STATUSES:
            bad = f"status {st} outside the reader's set"
        elif st == 0:
            cfg = {"n_embd": d.n_embd, "n_ff": d.n_ff, "n_head": d.n_head, "n_head_kv": d.n_head_kv,
                   "n_vocab": d.n_vocab}
            tensors = {"tok_embd": d.tok_embd - buf, "output_norm": d.output_norm - buf}
            for il in range(d.n_layer):
                for name in amd.LAYER_I2S + amd.LAYER_NORMS:
                    tensors[(il, name)] = getattr(layers[il], name) - buf
            for off, size in extents(cfg, tensors):
                if off < 0 or off + size > len(img):
                    bad = f"accepted, but a tensor's data [{off}, {off + size}) lies outside the {len(img)}-byte image"
                    break
        libc.free(buf)
        hist[st] = hist.get(st, 0) + 1
        n += 1
        if bad:
            print(f"gguf_fuzz: FINDING after {n} mutants: {bad}\n{img.hex()}", flush=True)
            sys.exit(1)
    print(f"gguf_fuzz: {n} mutants of {len(pool)} seeds in {seconds:.0f} s, seed {seed}, no finding; statuses "
          + ", ".join(f"{k}: {v}" for k, v in sorted(hist.items())), flush=True)


if __name__ == "__main__":
    main()

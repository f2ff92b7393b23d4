#!/usr/bin/env python3
"""Extract the reference's I2_S golden data into JSON fixtures.

Reads two data files the reference's own tests hold (they are upstream
captures, not saphira-llm output; tests/golden/README.md:1-30 there):

  tests/golden/i2s-converter.txt  -- 17 cases, each: n, the packed bytes
      (codes + f32 scale) under both upstream packing rules, and the values
      upstream's dequantize_row_i2_s decoded from them (independent read-back)
  tests/golden/i2s-reference.txt  -- 4 GEMV records captured from upstream
      ggml_gemv_i2_i8_s on real weights against the fixed LCG activation:
      n, act_scale, act_sum, w_scale, the first 16 raw int32 dots and the
      first 8 epilogue outputs, plus FNV-1a hashes over 512 rows

and writes i2s_converter.json / i2s_reference.json beside this script. Only
data moves: the fixtures hold inputs and expected outputs, nothing else.

    python3 tests/golden/make_fixtures.py [/root/reference]
"""
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))


def parse_converter(path):
    cases = []
    for line in open(path):
        if not line.startswith("case "):
            continue
        parts = [p.split() for p in line.rstrip("\n").split("|")]
        head = parts[0]
        n, nbytes, scale_hex = int(head[1]), int(head[2]), head[3]
        packed_c, decoded_c, packed_py, decoded_py, differ = parts[1:6]
        assert differ[0] == "differ"
        assert len(packed_c) == len(packed_py) == nbytes
        assert len(decoded_c) == len(decoded_py) == n
        cases.append({
            "n": n, "packed_bytes": nbytes, "scale_f32_hex": scale_hex,
            "rules": {
                "bitnet_c": {"packed_hex": "".join(packed_c), "decoded_f32_hex": decoded_c},
                "gguf_py": {"packed_hex": "".join(packed_py), "decoded_f32_hex": decoded_py},
            },
            "differ": int(differ[1]),
        })
    return cases


def parse_reference(path):
    records, cur = [], None
    for line in open(path):
        s = line.strip()
        if s.startswith("gemv "):
            cur = {"tensor": s.split()[1]}
            records.append(cur)
            continue
        if s.startswith("tensor ") or not s:
            cur = None if s.startswith("tensor ") else cur
            continue
        if cur is None:
            continue
        key, _, rest = s.partition(" ")
        if key in ("n", "rows", "act_sum", "gemv_gemm_agree"):
            cur[key] = int(rest)
        elif key in ("act_scale", "w_scale"):
            cur[key] = rest            # keep the printed decimal (%.9g), exact for f32
        elif key in ("fnv1a64", "epilogue_fnv1a64"):
            cur[key] = rest
        elif key == "values":
            cur[key] = [int(float(v)) for v in rest.split()]
        elif key == "epilogue_values":
            cur[key] = rest.split()    # printed with %f: compare as text
    return records


def main():
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    golden = os.path.join(ref, "tests", "golden")
    conv = parse_converter(os.path.join(golden, "i2s-converter.txt"))
    gem = parse_reference(os.path.join(golden, "i2s-reference.txt"))
    src = "saphira-llm tests/golden/%s (upstream capture)"
    with open(os.path.join(HERE, "i2s_converter.json"), "w") as f:
        json.dump({"source": src % "i2s-converter.txt", "cases": conv}, f, separators=(",", ":"))
    with open(os.path.join(HERE, "i2s_reference.json"), "w") as f:
        json.dump({"source": src % "i2s-reference.txt", "gemv": gem}, f, indent=1)
    print(f"{len(conv)} converter cases, {len(gem)} gemv records")


if __name__ == "__main__":
    main()

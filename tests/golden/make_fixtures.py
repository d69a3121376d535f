"""Writes the golden fixtures of tests/golden from the reference's own test data (run once, in a container where
/root/reference is mounted; the GPU box and the tests only read the committed JSON).

  mxfp4_reference.json  MXFP4ReferenceTests.words / scales / values (Tests/IngotTests/KernelCaseMXFP4.swift:142-158):
                        16 packed e2m1 words, 4 e8m0 scales and the 128 fp32 values mlx's mx.dequantize(mode="mxfp4")
                        gives for them (ref/mxfp4_ref.py), including -0.
  router_vectors.json   ref/router_vectors.json (written by mlx-lm 0.32.2's router code, ref/router_ref.py), copied as
                        data: per case E, top-k, scoring, logits, biases and mlx-lm's dense routing weights.
  rope_ref.json         ref/rope/rope_ref.json (mlx-lm initialize_rope, ref/rope_ref.py), copied as data: per case θ,
                        rotated dims, the RoPE parameter dict, mlx-lm's fp32 inv_freq, the same formula in float64 and
                        mscale (yarn-truncate, gpt-oss, yarn-mscale, linear, default).
"""
import json
import re
import struct
from pathlib import Path

REF = Path("/root/reference")
OUT = Path(__file__).resolve().parent


def swift_array(text: str, name: str) -> str:
    m = re.search(r"static let " + name + r"\s*:\s*\[[A-Za-z0-9]+\]\s*=\s*\[(.*?)\]", text, re.S)
    if not m:
        raise SystemExit(f"{name} not found")
    return m.group(1)


def main() -> None:
    src = (REF / "Tests/IngotTests/KernelCaseMXFP4.swift").read_text()
    words = [int(w.replace("_", ""), 16) for w in re.findall(r"0x[0-9A-Fa-f_]+", swift_array(src, "words"))]
    scales = [int(s) for s in re.findall(r"\d+", swift_array(src, "scales"))]
    vals_txt = [v.strip() for v in swift_array(src, "values").split(",") if v.strip()]
    values = [float(v) for v in vals_txt]
    # Keep the sign of zero as bit patterns (JSON has no -0 for integers, and float -0.0 is kept by json, but the
    # bits are explicit).
    bits = [struct.unpack("<I", struct.pack("<f", v))[0] for v in values]
    assert len(words) == 16 and len(scales) == 4 and len(values) == 128
    (OUT / "mxfp4_reference.json").write_text(json.dumps(
        {"source": "Tests/IngotTests/KernelCaseMXFP4.swift:142-158 (mlx mx.dequantize mode=mxfp4, ref/mxfp4_ref.py)",
         "rows": 2, "cols": 64, "words": words, "scales": scales, "values": values, "value_bits": bits}, indent=1))
    rv = json.loads((REF / "ref/router_vectors.json").read_text())
    rv["copied_from"] = "ref/router_vectors.json"
    (OUT / "router_vectors.json").write_text(json.dumps(rv))
    rr = json.loads((REF / "ref/rope/rope_ref.json").read_text())
    (OUT / "rope_ref.json").write_text(json.dumps({"copied_from": "ref/rope/rope_ref.json", "cases": rr}))
    print("wrote", OUT / "mxfp4_reference.json", OUT / "router_vectors.json", OUT / "rope_ref.json")


if __name__ == "__main__":
    main()

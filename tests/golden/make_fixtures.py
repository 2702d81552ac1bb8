"""Writes the golden fixtures the oracle tests read, from the data files the reference's own tests hold:

- mlx_affine4.json, mlx_affine8.json: the 4-bit and 8-bit MLX affine entries (groups 32, 64, 128) of the
  reference's dev/tests/fixtures/mlx-quantization/fixture.json, which MLX 0.32.3 wrote
  (dev/tools/mlx_quantization_fixture.py): packed weight, bf16 scales and biases, codes, and MLX's fp32 values
  fma(code, s, z), all hex.
- weight_goldens.json: the Q4_K, Q5_K, Q6_K and Q8_0 SHA-256 of dev/tests/fixtures/weight-goldens/goldens.json
  (gguf_dequantization), llama.cpp 7ab4ee7's fp32 dequantisation of fixture(format, 256 rows, 1024 columns,
  mt19937 seed 7 + format id) (gguf_reference_test.mm:20-25).

Both are copied as data. Usage: python tests/golden/make_fixtures.py /path/to/reference
"""
import json
import pathlib
import sys

reference = pathlib.Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
here = pathlib.Path(__file__).resolve().parent
mlx = json.loads((reference / "dev/tests/fixtures/mlx-quantization/fixture.json").read_text())
for bits in (4, 8):
    entries = [f for f in mlx["formats"] if f["mode"] == "affine" and f["bits"] == bits]
    (here / f"mlx_affine{bits}.json").write_text(json.dumps({
        "source": "splash-desktop dev/tests/fixtures/mlx-quantization/fixture.json (MLX %s)" % mlx["mlx"],
        "formats": entries}, indent=1) + "\n")
goldens = json.loads((reference / "dev/tests/fixtures/weight-goldens/goldens.json").read_text())
(here / "weight_goldens.json").write_text(json.dumps({
    "source": "splash-desktop dev/tests/fixtures/weight-goldens/goldens.json (llama.cpp 7ab4ee7)",
    "fixture": {"format": "q4k", "rows": 256, "columns": 1024, "seed": 7},
    "q4k": goldens["gguf_dequantization"]["q4k"],
    "formats": {name: {"id": fid, "seed": 7 + fid, "sha256": goldens["gguf_dequantization"][name]}
                for name, fid in (("q4k", 0), ("q5k", 3), ("q6k", 4), ("q80", 6))}}, indent=1) + "\n")
print("wrote the MLX entries and the Q4_K, Q5_K, Q6_K and Q8_0 goldens")

"""Writes the golden fixtures the oracle tests read, from the data files the reference's own tests hold:

- mlx_affine4.json: the 4-bit MLX affine entries (groups 32, 64, 128) of the reference's
  dev/tests/fixtures/mlx-quantization/fixture.json, which MLX 0.32.3 wrote (dev/tools/mlx_quantization_fixture.py):
  packed weight, bf16 scales and biases, codes, and MLX's fp32 values fma(code, s, z), all hex.
- weight_goldens.json: the Q4_K SHA-256 of dev/tests/fixtures/weight-goldens/goldens.json (gguf_dequantization.q4k),
  llama.cpp 7ab4ee7's fp32 dequantisation of fixture(Q4_K, 256 rows, 1024 columns, mt19937 seed 7).

Both are copied as data. Usage: python tests/golden/make_fixtures.py /path/to/reference
"""
import json
import pathlib
import sys

reference = pathlib.Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
here = pathlib.Path(__file__).resolve().parent
mlx = json.loads((reference / "dev/tests/fixtures/mlx-quantization/fixture.json").read_text())
entries = [f for f in mlx["formats"] if f["mode"] == "affine" and f["bits"] == 4]
(here / "mlx_affine4.json").write_text(json.dumps({
    "source": "splash-desktop dev/tests/fixtures/mlx-quantization/fixture.json (MLX %s)" % mlx["mlx"],
    "formats": entries}, indent=1) + "\n")
goldens = json.loads((reference / "dev/tests/fixtures/weight-goldens/goldens.json").read_text())
(here / "weight_goldens.json").write_text(json.dumps({
    "source": "splash-desktop dev/tests/fixtures/weight-goldens/goldens.json (llama.cpp 7ab4ee7)",
    "fixture": {"format": "q4k", "rows": 256, "columns": 1024, "seed": 7},
    "q4k": goldens["gguf_dequantization"]["q4k"]}, indent=1) + "\n")
print("wrote", len(entries), "MLX entries and the Q4_K golden")

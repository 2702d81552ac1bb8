// Driver over the reference's own CPU oracle, dev/tests/engine/GgufFormatReference.hpp (with the headers it
// includes: runtime/metal/abi/QuantFormat.h, QuantTables.h, dev/tests/engine/LinearNumerics.hpp), compiled from
// where those files lie in the reference checkout into oracle/_ref/libsqref.so (oracle/Makefile). TEST
// INFRASTRUCTURE ONLY: it exports C entry points so the tests can check the C restatement (sq_oracle.c) against
// the reference's repack, values and bounds on the same inputs. Nothing here is part of the product.
#include "GgufFormatReference.hpp"

#include <cstring>
#include <random>

using namespace gguf_reference;

extern "C" {

// repack(f, native, N, K, &values) (GgufFormatReference.hpp:701-725): plane0, meta and the fp32 values.
int sqref_repack(uint32_t fmt, const uint8_t *native, uint32_t N, uint32_t K, uint8_t *plane0, uint8_t *meta,
                 float *values) {
  try {
    const std::vector<uint8_t> in(native, native + size_t(N) * rowBytes(Fmt(fmt), K));
    std::vector<float> v;
    const Packed p = repack(Fmt(fmt), in, N, K, &v);
    std::memcpy(plane0, p.w0.data(), p.w0.size());
    std::memcpy(meta, p.meta.data(), p.meta.size());
    std::memcpy(values, v.data(), v.size() * sizeof(float));
    return 0;
  } catch (...) {
    return -1;
  }
}

// repack with plane1 as well (formats with high bits: Q5_K, Q6_K).
int sqref_repack_planes(uint32_t fmt, const uint8_t *native, uint32_t N, uint32_t K, uint8_t *plane0,
                        uint8_t *plane1, uint8_t *meta, float *values) {
  try {
    const std::vector<uint8_t> in(native, native + size_t(N) * rowBytes(Fmt(fmt), K));
    std::vector<float> v;
    const Packed p = repack(Fmt(fmt), in, N, K, &v);
    std::memcpy(plane0, p.w0.data(), p.w0.size());
    if (plane1 && kQuantFormats[fmt].plane1_bytes) std::memcpy(plane1, p.w1.data(), p.w1.size());
    std::memcpy(meta, p.meta.data(), p.meta.size());
    std::memcpy(values, v.data(), v.size() * sizeof(float));
    return 0;
  } catch (...) {
    return -1;
  }
}

// The test fixture of GgufFixtures.hpp:148-165 through the reference's makeNative (GgufFixtures.hpp itself needs
// Foundation, so its three-line scale draw is restated here and handed to makeNative).
int sqref_fixture(uint32_t fmt, uint32_t rows, uint32_t K, uint32_t seed, uint8_t *native) {
  std::mt19937 rng(seed);
  const Fmt f = Fmt(fmt);
  std::vector<uint8_t> v;
  if (affine(f)) {
    v.resize(size_t(rows) * rowBytes(f, K));
    for (auto &b : v) b = uint8_t(rng());
    for (size_t at = 0; at < v.size(); at += kQuantFormats[f].block_bytes)
      for (size_t field = 0; field < 4; field += 2)
        if ((v[at + field + 1] & 0x7F) == 0x7F && (v[at + field] & 0x80)) v[at + field + 1] ^= 1;
  } else {
    v = makeNative(f, rows, K, rng, [&] {
      uint16_t h;
      do h = static_cast<uint16_t>(rng());
      while ((h & 0x7C00) == 0x7C00);
      return h;
    });
  }
  std::memcpy(native, v.data(), v.size());
  return 0;
}

// mlxNative (GgufFormatReference.hpp:236-270).
int sqref_mlx_native(uint32_t fmt, uint32_t rows, uint32_t K, const uint8_t *weight, const uint8_t *scales,
                     const uint8_t *biases, uint8_t *native) {
  const Fmt f = Fmt(fmt);
  const uint32_t groups = K / kQuantFormats[f].block_elements;
  const std::vector<uint8_t> w(weight, weight + size_t(rows) * K / 2), s(scales, scales + size_t(rows) * groups * 2),
      b(biases, biases + size_t(rows) * groups * 2);
  const std::vector<uint8_t> out = mlxNative(f, rows, K, w, s, b);
  std::memcpy(native, out.data(), out.size());
  return 0;
}

// projectionBound (GgufFormatReference.hpp:794-797) of a dot's magnitudes.
double sqref_projection_bound(double magnitude, double inputs, double largest, int staged) {
  Dot d;
  d.magnitude = magnitude;
  d.inputs = inputs;
  d.largest = largest;
  return projectionBound(d, staged != 0);
}

uint32_t sqref_quant_slot(uint32_t e) { return quant_slot(e); }
uint64_t sqref_tile_index(uint32_t row, uint32_t block, uint32_t blocks) { return quant_tile_index(row, block, blocks); }
int sqref_format_row(uint32_t fmt, uint32_t out[7]) {
  if (fmt >= GGUF_FMT_COUNT) return -1;
  const QuantFormat &q = kQuantFormats[fmt];
  const uint32_t row[7] = {q.ggml_type, q.block_elements, q.block_bytes, q.plane0_bytes, q.plane1_bytes, q.meta_bytes,
                           q.meta_groups};
  std::memcpy(out, row, sizeof row);
  return 0;
}
uint16_t sqref_f2h(float f) { return f2h(f); }

}  // extern "C"

// Host-side table producers of the INT8 attention path.
//
// h3_rope_dit_tables restates rope::dit (reference src/rope.rs:11-37), the producer of the
// cos/sin tables that h3_prepare_qk_rope_i8hm and h3_rope_qknorm_f16 read. It stays on the host,
// as in the reference (src/layout.rs:66-73): the tables are built once per sequence layout and
// uploaded with the other per-layout buffers.
#include <cmath>
#include <cstring>
#include <unordered_map>

#include "internal.hpp"

namespace {

constexpr int kAxes = 3;
constexpr int kFreqs = 16;                   // frequencies per axis
constexpr int kRopeHalf = kAxes * kFreqs;    // 48 table entries per token (model.rs ROPE_HALF)

struct AxisRow {
  float c[kFreqs];
  float s[kFreqs];
};

}  // namespace

extern "C" int h3_rope_dit_tables(const double* pos, size_t rows, const float* inv_freq,
                                  float* cos_t, float* sin_t) {
  const char* stage = "rope_dit_tables";
  if (rows == 0) {
    h3::set_error(H3_OK, "%s", "");
    return H3_OK;
  }
  if (!pos || !inv_freq || !cos_t || !sin_t)
    return h3::set_error(H3_ERR_ARGUMENT, "%s: null pointer", stage);
  // Rows repeat the same axis coordinates; cache each coordinate after its narrowing to float,
  // keyed by its bits so -0.0 and 0.0 stay distinct (their sines differ in sign).
  std::unordered_map<uint32_t, AxisRow> axes;
  for (size_t r = 0; r < rows; ++r) {
    for (int ax = 0; ax < kAxes; ++ax) {
      const float p = static_cast<float>(pos[kAxes * r + ax]);
      uint32_t key;
      std::memcpy(&key, &p, sizeof key);
      auto it = axes.find(key);
      if (it == axes.end()) {
        AxisRow row;
        for (int j = 0; j < kFreqs; ++j) {
          const float angle = p * inv_freq[j];  // float angle: cosf, not cos narrowed
          row.c[j] = std::cos(angle);
          row.s[j] = std::sin(angle);
        }
        it = axes.emplace(key, row).first;
      }
      const size_t start = r * kRopeHalf + ax * kFreqs;
      std::memcpy(cos_t + start, it->second.c, sizeof it->second.c);
      std::memcpy(sin_t + start, it->second.s, sizeof it->second.s);
    }
  }
  h3::set_error(H3_OK, "%s", "");
  return H3_OK;
}

// Host RoPE table builder (replaces RopeTable, /root/reference/src/cuda/inference.cu:
// 764-785).  Same float/double mix and evaluation order as the reference so the BF16
// entries are bit-identical on the same libm; theta, head_dim and the YaRN constants
// are parameters.  Built with -ffp-contract=off.
#include <cmath>
#include <cstdint>
#include <cstring>

#include "padra_hip.h"

namespace {
uint16_t ToBF16(float x) {  // RNE, as BHost (inference.cu:742-748)
  std::uint32_t bits;
  std::memcpy(&bits, &x, 4);
  if ((bits & 0x7fffffffu) > 0x7f800000u)
    return 0x7fffu;
  bits += 0x7fffu + ((bits >> 16) & 1u);
  return static_cast<uint16_t>(bits >> 16);
}
}  // namespace

extern "C" int padra_RopeTable(uint16_t *table, int positions, int head_dim, float theta,
                               int yarn, float factor, int original_context) {
  if (!table || positions < 1 || head_dim < 2 || head_dim % 2 || head_dim > 1024 ||
      !(theta > 1.f) || (yarn && (!(factor > 0.f) || original_context < 1)))
    return PADRA_INVALID_ARGUMENT;
  const int half = head_dim / 2;
  const double pi = std::acos(-1.0), base = static_cast<double>(theta);
  const float low = static_cast<float>(std::fmax(
      0., std::floor(head_dim * std::log(original_context / (32 * 2 * pi)) / (2 * std::log(base)))));
  const float high = static_cast<float>(std::fmin(
      static_cast<double>(head_dim - 1),
      std::ceil(head_dim * std::log(original_context / (2 * pi)) / (2 * std::log(base)))));
  float frequencies[512];
  for (int i = 0; i < half; ++i) {
    const float freq = powf(theta, static_cast<float>(2 * i) / static_cast<float>(head_dim));
    float ramp = (static_cast<float>(i) - low) / (high - low);
    ramp = ramp < 0.f ? 0.f : (ramp > 1.f ? 1.f : ramp);
    const float extra = 1 - ramp;
    frequencies[i] = !yarn ? 1 / freq : (1 / (factor * freq)) * (1 - extra) + (1 / freq) * extra;
  }
  const float scale = !yarn ? 1.f : static_cast<float>(1 + 0.1 * std::log(static_cast<double>(factor)));
  for (int p = 0; p < positions; ++p)
    for (int i = 0; i < half; ++i) {
      const float angle = static_cast<float>(p) * frequencies[i];
      table[static_cast<long long>(p) * head_dim + i] = ToBF16(cosf(angle) * scale);
      table[static_cast<long long>(p) * head_dim + half + i] = ToBF16(sinf(angle) * scale);
    }
  return PADRA_OK;
}

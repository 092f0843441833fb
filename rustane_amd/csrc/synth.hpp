// Seeded synthetic weights and tokens, identical on host and device.
//
// Each value is a pure function of (seed, tensor id, element index): a
// counter-based hash (splitmix64 finaliser) gives 128 random bits per element;
// the eight 16-bit fields are summed as integers, centred, and scaled once in
// fp32. The sum of eight uniforms (Irwin-Hall, n = 8) is a close normal
// approximation (excess kurtosis -0.15) with exactly the requested standard
// deviation. All steps before the single fp32 multiply are exact integer
// arithmetic, so host and device produce bit-identical floats.
#pragma once
#include <stdint.h>
#include <math.h>

#if defined(__HIPCC__)
#define HB_HD __host__ __device__ inline
#else
#define HB_HD inline
#endif

HB_HD uint64_t hb_mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

HB_HD uint64_t hb_stream_key(uint64_t seed, uint64_t stream) {
  return hb_mix64(seed * 0x9E3779B97F4A7C15ull ^ (stream + 0x632BE59BD9B4E019ull) * 0xC2B2AE3D27D4EB4Full);
}

HB_HD uint64_t hb_hash(uint64_t key, uint64_t i) { return hb_mix64(key + i * 0x9E3779B97F4A7C15ull); }

// Integer part of the normal sample: sum of 8 uniform 16-bit draws minus the mean.
HB_HD int32_t hb_irwin_hall8(uint64_t key, uint64_t i) {
  const uint64_t a = hb_hash(key, 2 * i), b = hb_hash(key, 2 * i + 1);
  int32_t s = 0;
  for (int j = 0; j < 4; ++j) {
    s += (int32_t)((a >> (16 * j)) & 0xFFFFu);
    s += (int32_t)((b >> (16 * j)) & 0xFFFFu);
  }
  return s - 262140;  // 8 * 65535 / 2
}

// fp32 scale that maps the integer sum to standard deviation `std`.
inline float hb_normal_scale(float std) {
  const double sd = sqrt(8.0 * (65536.0 * 65536.0 - 1.0) / 12.0);
  return (float)((double)std / sd);
}

HB_HD float hb_normal_value(uint64_t key, uint64_t i, float scale) {
  return (float)hb_irwin_hall8(key, i) * scale;
}

HB_HD uint32_t hb_token_value(uint64_t key, uint64_t i, uint32_t vocab) {
  return (uint32_t)(((hb_hash(key, i) >> 32) * (uint64_t)vocab) >> 32);
}

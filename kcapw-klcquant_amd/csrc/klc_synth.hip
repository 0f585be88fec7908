// Counter-based SplitMix64 fill, identical to klcquant_amd/synth.py: element i
// uses draw(seed, i) = mix64(mix64(seed) + (i + 1) * GAMMA).
#include "klc_common.h"

namespace klc {
namespace {

constexpr uint64_t kGamma = 0x9E3779B97F4A7C15ull;

__host__ __device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// mode 0: bytes of the little-endian words draw(i); mode 1: one byte per draw in [lo, hi].
__global__ __launch_bounds__(256) void synth_fill_kernel(uint8_t* __restrict__ dst, int64_t n, uint64_t state,
                                                         int mode, int lo, int span) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  if (mode == 0) {
    const int64_t words = (n + 7) / 8;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < words; i += stride) {
      const uint64_t z = mix64(state + (uint64_t)(i + 1) * kGamma);
      if ((i + 1) * 8 <= n) {
        reinterpret_cast<uint64_t*>(dst)[i] = z;
      } else {
        for (int64_t b = i * 8; b < n; ++b) dst[b] = (uint8_t)(z >> (8 * (b - i * 8)));
      }
    }
  } else {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
      const uint64_t z = mix64(state + (uint64_t)(i + 1) * kGamma);
      dst[i] = (uint8_t)(lo + (int)(((z >> 32) * (uint64_t)span) >> 32));
    }
  }
}

}  // namespace
}  // namespace klc

using namespace klc;

extern "C" int klc_synth_fill(void* dst, int64_t n, uint64_t seed, int mode, int lo, int hi, void* stream) {
  KLC_REQUIRE(dst, KLC_ERR_ARGUMENT, "klc_synth_fill: null pointer");
  KLC_REQUIRE(n >= 0, KLC_ERR_ARGUMENT, "klc_synth_fill: n=%lld", (long long)n);
  KLC_REQUIRE(mode == 0 || mode == 1, KLC_ERR_ARGUMENT, "klc_synth_fill: mode=%d", mode);
  if (mode == 0) {
    KLC_REQUIRE(((uintptr_t)dst & 7) == 0, KLC_ERR_ARGUMENT, "klc_synth_fill: dst must be 8-byte aligned");
  } else {
    KLC_REQUIRE(0 <= lo && lo <= hi && hi <= 255, KLC_ERR_ARGUMENT, "klc_synth_fill: bad range [%d, %d]", lo, hi);
  }
  if (n == 0) return KLC_OK;
  const int64_t items = mode == 0 ? (n + 7) / 8 : n;
  const int64_t want = (items + 255) / 256;
  const unsigned grid = (unsigned)(want < 16384 ? want : 16384);
  synth_fill_kernel<<<grid, 256, 0, as_stream(stream)>>>(static_cast<uint8_t*>(dst), n, mix64(seed), mode, lo,
                                                         hi - lo + 1);
  return check_launch("synth_fill_kernel");
}

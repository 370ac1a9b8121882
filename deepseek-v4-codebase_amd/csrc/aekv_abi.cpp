// Library-level C ABI of libaetherkv: version, error reporting, limits and the host-side
// Rademacher diagonal.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>

#include "aekv_common.h"

namespace aekv {

namespace {
thread_local char g_last_error[512] = {0};

// MT19937 (Matsumoto & Nishimura 1998): the generator behind torch.rand on the CPU.
struct Mt19937 {
  uint32_t mt[624];
  int idx;
  explicit Mt19937(uint32_t s) {
    mt[0] = s;
    for (int i = 1; i < 624; ++i) mt[i] = 1812433253u * (mt[i - 1] ^ (mt[i - 1] >> 30)) + static_cast<uint32_t>(i);
    idx = 624;
  }
  uint32_t next() {
    if (idx >= 624) {
      for (int i = 0; i < 624; ++i) {
        const uint32_t y = (mt[i] & 0x80000000u) | (mt[(i + 1) % 624] & 0x7fffffffu);
        mt[i] = mt[(i + 397) % 624] ^ (y >> 1) ^ ((y & 1u) ? 0x9908b0dfu : 0u);
      }
      idx = 0;
    }
    uint32_t y = mt[idx++];
    y ^= y >> 11;
    y ^= (y << 7) & 0x9d2c5680u;
    y ^= (y << 15) & 0xefc60000u;
    y ^= y >> 18;
    return y;
  }
};
}  // namespace

int fail(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return status;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(AEKV_ERR_HIP, "%s: HIP error %d (%s)", what, static_cast<int>(e), hipGetErrorString(e));
  return AEKV_OK;
}

float wht_scale(int d) { return static_cast<float>(std::pow(static_cast<double>(d), -0.5)); }

}  // namespace aekv

extern "C" const char* aekv_version(void) { return "aetherkv 0.1.0 gfx950"; }

extern "C" const char* aekv_last_error(void) { return aekv::g_last_error; }

extern "C" int32_t aekv_max_head_dim(void) { return 512; }

extern "C" int32_t aekv_max_topk(void) { return 2048; }

// PolarQuant._diag (aether_2b/turbo_quant.py:111-121): Generator().manual_seed(seed*10007+d);
// torch.rand(d) draws (u32 & 0xFFFFFF) * 2^-24 from MT19937 seeded with the low 32 bits.
extern "C" int aekv_tq_diag(int64_t seed, int32_t d, float* out_host) {
  if (d <= 0) return aekv::fail(AEKV_ERR_VALUE, "aekv_tq_diag: d must be positive, got %d", d);
  if (!out_host) return aekv::fail(AEKV_ERR_VALUE, "aekv_tq_diag: null output");
  aekv::Mt19937 g(static_cast<uint32_t>(static_cast<uint64_t>(seed * 10007 + d) & 0xffffffffu));
  for (int i = 0; i < d; ++i) {
    const float r = static_cast<float>(g.next() & 0xffffffu) * 0x1p-24f;
    out_host[i] = r > 0.5f ? 1.0f : -1.0f;
  }
  return AEKV_OK;
}

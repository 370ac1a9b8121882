// Streaming ceilings for the traffic of two kernels: measurement utilities for bench.py with no
// counterpart in the reference, built into their own library (libaetherkv_probe.so, declared in
// include/aetherkv_probe.h) so that the product library exports only the path's entry points.
//
// stream_probe_kernel moves exactly the encode's bytes with the encode's access pattern and
// almost no arithmetic: one wave per group of 16 vectors of 128 bf16 (lane 4v + g reads the 64
// bytes [64 g, 64 g + 64) of vector v), 16 bytes out per lane (the 4-bit codes' 64 bytes per
// vector) and 4 bytes per vector (the scale), both with non-temporal stores.  The outputs are xor
// folds of the inputs, so no load can be dropped.  Its time is the box's practical HBM ceiling
// for this stream, beside the 8 TB/s datasheet peak.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "aetherkv_probe.h"

namespace {

typedef __attribute__((ext_vector_type(4))) uint32_t u32x4_t;

__global__ __launch_bounds__(256) void stream_probe_kernel(const uint4* __restrict__ x, int64_t n_vec,
                                                           uint4* __restrict__ codes, float* __restrict__ scale) {
  const int lane = threadIdx.x & 63;
  const int v = lane >> 2, g = lane & 3;
  const int64_t grp = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int64_t n_groups = (n_vec + 15) >> 4;
  if (grp >= n_groups) return;
  const int64_t rem = n_vec - grp * 16;
  const uint32_t vv = static_cast<uint32_t>(v < rem ? v : rem - 1);
  const char* base = reinterpret_cast<const char*>(x + grp * 256) + vv * 256u + static_cast<uint32_t>(g) * 64u;
  uint4 t[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) t[i] = *reinterpret_cast<const uint4*>(base + 16 * i);
  const u32x4_t o = {t[0].x ^ t[1].x ^ t[2].x ^ t[3].x, t[0].y ^ t[1].y ^ t[2].y ^ t[3].y,
                     t[0].z ^ t[1].z ^ t[2].z ^ t[3].z, t[0].w ^ t[1].w ^ t[2].w ^ t[3].w};
  if (v < rem) {
    if (g == 0)
      __builtin_nontemporal_store(__builtin_bit_cast(float, o.x ^ o.y), scale + grp * 16 + v);
    __builtin_nontemporal_store(o, reinterpret_cast<u32x4_t*>(codes + grp * 64) + 4 * v + g);
  }
}

// scan_probe_kernel: the CSA score pass's traffic with no arithmetic.  One wave per group of 128
// keys of one row (the score kernel's decode group at 4 bits): the group's code bytes (128 x RB,
// 16 bytes per lane and load) and its 128 scales (8 bytes per lane) are read, and, with keys set, 4
// bytes per key (8 per lane) and 4 per 16-key slot are written, as the order keys and slot maxima.
// The written values are xor folds of the loaded ones, so no load can be dropped.
template <int RB>
__global__ __launch_bounds__(256) void scan_probe_kernel(const uint4* __restrict__ codes, const uint2* __restrict__ scale,
                                                         int64_t n_groups, uint2* __restrict__ keys,
                                                         uint32_t* __restrict__ smax) {
  constexpr int kLoads = 128 * RB / 16 / 64;  // 16-byte loads per lane
  const int lane = threadIdx.x & 63;
  const int64_t grp = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (grp >= n_groups) return;
  const uint4* c = codes + grp * (128 * RB / 16);
  uint4 t[kLoads];
#pragma unroll
  for (int i = 0; i < kLoads; ++i) t[i] = c[64 * i + lane];
  const uint2 sc = scale[grp * 64 + lane];
  uint32_t x = sc.x, y = sc.y;
#pragma unroll
  for (int i = 0; i < kLoads; ++i) {
    x ^= t[i].x ^ t[i].z;
    y ^= t[i].y ^ t[i].w;
  }
  if (keys) {
    keys[grp * 64 + lane] = make_uint2(x, y);
    if ((lane & 7) == 0) smax[grp * 8 + (lane >> 3)] = x + y;
  } else if (x == 0x9e3779b9u && y == 0x7f4a7c15u) {
    smax[0] = x;  // (never in practice: keeps the loads live)
  }
}

}  // namespace

extern "C" int aekv_scan_probe(const void* codes, const float* scale, int64_t n_keys, int32_t row_bytes, void* keys,
                               uint32_t* smax, void* stream) {
  auto aligned = [](const void* p, uintptr_t a) { return reinterpret_cast<uintptr_t>(p) % a == 0; };
  if (n_keys < 0 || n_keys % 128 != 0 || (row_bytes != 32 && row_bytes != 64)) return AEKV_PROBE_ERR_ARGS;
  if (n_keys == 0) return AEKV_PROBE_OK;
  if (!codes || !scale || !smax || !aligned(codes, 16) || !aligned(scale, 8) || (keys && !aligned(keys, 8)) ||
      !aligned(smax, 4))
    return AEKV_PROBE_ERR_ARGS;
  const int64_t n_groups = n_keys / 128;
  const int64_t blocks = (n_groups + 3) / 4;
  if (blocks > 0x7fffffff) return AEKV_PROBE_ERR_ARGS;
  auto fn = row_bytes == 32 ? scan_probe_kernel<32> : scan_probe_kernel<64>;
  hipLaunchKernelGGL(fn, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                     static_cast<const uint4*>(codes), reinterpret_cast<const uint2*>(scale), n_groups,
                     static_cast<uint2*>(keys), smax);
  return hipGetLastError() == hipSuccess ? AEKV_PROBE_OK : AEKV_PROBE_ERR_LAUNCH;
}

extern "C" int aekv_stream_probe(const void* x, int64_t n_vec, void* codes, float* scale, void* stream) {
  auto aligned = [](const void* p, uintptr_t a) { return reinterpret_cast<uintptr_t>(p) % a == 0; };
  if (n_vec < 0) return AEKV_PROBE_ERR_ARGS;
  if (n_vec == 0) return AEKV_PROBE_OK;
  if (!x || !codes || !scale || !aligned(x, 16) || !aligned(codes, 16) || !aligned(scale, 4))
    return AEKV_PROBE_ERR_ARGS;
  const int64_t blocks = ((n_vec + 15) / 16 + 3) / 4;
  if (blocks > 0x7fffffff) return AEKV_PROBE_ERR_ARGS;
  hipLaunchKernelGGL(stream_probe_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), static_cast<const uint4*>(x), n_vec,
                     static_cast<uint4*>(codes), scale);
  return hipGetLastError() == hipSuccess ? AEKV_PROBE_OK : AEKV_PROBE_ERR_LAUNCH;
}

// Streaming ceiling for the cfg2 encode's traffic shape (a measurement utility for bench.py; no
// counterpart in the reference).
//
// stream_probe_kernel moves exactly the encode's bytes with the encode's access pattern and
// almost no arithmetic: one wave per group of 16 vectors of 128 bf16 (lane 4v + g reads the 64
// bytes [64 g, 64 g + 64) of vector v), 16 bytes out per lane (the 4-bit codes' 64 bytes per
// vector) and 4 bytes per vector (the scale), both with non-temporal stores.  The outputs are xor
// folds of the inputs, so no load can be dropped.  Its time is the box's practical HBM ceiling
// for this stream, beside the 8 TB/s datasheet peak.
#include "aekv_common.h"

namespace aekv {
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

}  // namespace
}  // namespace aekv

using namespace aekv;

extern "C" int aekv_stream_probe(const void* x, int64_t n_vec, void* codes, float* scale, void* stream) {
  const char* who = "aekv_stream_probe";
  if (n_vec < 0) return fail(AEKV_ERR_SHAPE, "%s: negative size", who);
  if (n_vec == 0) return AEKV_OK;
  if (!x || !codes || !scale) return fail(AEKV_ERR_VALUE, "%s: null pointer", who);
  if (!is_aligned(x, 16) || !is_aligned(codes, 16) || !is_aligned(scale, 4))
    return fail(AEKV_ERR_ALIGN, "%s: misaligned pointer", who);
  const int64_t blocks = ceil_div(ceil_div(n_vec, 16), 4);
  if (blocks > 0x7fffffff) return fail(AEKV_ERR_UNSUPPORTED, "%s: too many vectors", who);
  hipLaunchKernelGGL(stream_probe_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, as_stream(stream),
                     static_cast<const uint4*>(x), n_vec, static_cast<uint4*>(codes), scale);
  return check_launch(who);
}

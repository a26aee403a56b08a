// Probes for the measured roofline denominators (no reference counterpart; used by
// bench.py beside the published MI355X peaks):
//   motif_probe_copy       dst = src, nontemporal 16-byte loads and stores, a contiguous
//                          block per workgroup, eight loads in flight per thread: the HBM
//                          rate of a stream that reads and writes every byte once;
//   motif_probe_read       a reduction of src to one word per workgroup (nontemporal
//                          16-byte loads, eight in flight per thread): the read-only rate;
//   motif_probe_mfma_bf16  v_mfma_f32_16x16x32_bf16 (eight independent accumulators per
//                          wave) or v_mfma_f32_32x32x16_bf16 (four) back to back on register
//                          operands: the dense bf16 MFMA rate.
// Every probe writes a result that depends on all of its work, so nothing is elided.
#include "capi_internal.h"
#include "common.h"

namespace motif {

namespace {

constexpr int kProbeThreads = 256;

// 16-byte accesses marked nontemporal (the probed data is touched once)
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld_nt(const uint4 *p) {
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
  return uint4{v.x, v.y, v.z, v.w};
}
__device__ __forceinline__ void st_nt(uint4 v, uint4 *p) {
  __builtin_nontemporal_store(u32x4{v.x, v.y, v.z, v.w}, reinterpret_cast<u32x4 *>(p));
}

constexpr int kProbeUnroll = 8;  // 16-byte loads in flight per thread

// Each workgroup copies one contiguous block (a grid-stride interleave over all
// workgroups keeps many more DRAM pages open at once and measured ~20% slower).
__global__ void __launch_bounds__(kProbeThreads) probe_copy_kernel(const uint4 *src, uint4 *dst, size_t n) {
  const size_t per = n / gridDim.x, base = static_cast<size_t>(blockIdx.x) * per;
  const size_t end = blockIdx.x + 1 == gridDim.x ? n : base + per;
  size_t i = base + threadIdx.x;
  for (; i + (kProbeUnroll - 1) * kProbeThreads < end; i += kProbeUnroll * kProbeThreads) {
    uint4 v[kProbeUnroll];
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) v[u] = ld_nt(src + i + u * kProbeThreads);
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) st_nt(v[u], dst + i + u * kProbeThreads);
  }
  for (; i < end; i += kProbeThreads) dst[i] = src[i];
}

__global__ void __launch_bounds__(kProbeThreads) probe_read_kernel(const uint4 *src, uint32_t *out, size_t n) {
  const size_t stride = static_cast<size_t>(gridDim.x) * kProbeThreads;
  uint32_t acc = 0;
  size_t i = static_cast<size_t>(blockIdx.x) * kProbeThreads + threadIdx.x;
  for (; i + (kProbeUnroll - 1) * stride < n; i += kProbeUnroll * stride) {
    uint4 v[kProbeUnroll];
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) v[u] = ld_nt(src + i + u * stride);
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  for (; i < n; i += stride) {
    const uint4 a = src[i];
    acc ^= a.x ^ a.y ^ a.z ^ a.w;
  }
  __shared__ uint32_t red[kProbeThreads / 64];
  for (int off = 32; off > 0; off >>= 1) acc ^= __shfl_xor(acc, off, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t r = 0;
    for (int w = 0; w < kProbeThreads / 64; ++w) r ^= red[w];
    out[blockIdx.x] = r;
  }
}

__global__ void __launch_bounds__(kProbeThreads) probe_mfma_kernel(float *out, int iters, float seed) {
  const int lane = threadIdx.x & 63;
  bf16x8 a, b;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a[i] = static_cast<__bf16>(seed * static_cast<float>(lane + i));
    b[i] = static_cast<__bf16>(seed * static_cast<float>(lane - i));
  }
  f32x4 acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[j], 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) s += acc[j][0] + acc[j][1] + acc[j][2] + acc[j][3];
  out[static_cast<size_t>(blockIdx.x) * kProbeThreads + threadIdx.x] = s;
}

__global__ void __launch_bounds__(kProbeThreads) probe_mfma32_kernel(float *out, int iters, float seed) {
  const int lane = threadIdx.x & 63;
  bf16x8 a, b;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a[i] = static_cast<__bf16>(seed * static_cast<float>(lane + i));
    b[i] = static_cast<__bf16>(seed * static_cast<float>(lane - i));
  }
  typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
  f32x16 acc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[j][e] = 0.f;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[j], 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int e = 0; e < 16; ++e) s += acc[j][e];
  out[static_cast<size_t>(blockIdx.x) * kProbeThreads + threadIdx.x] = s;
}

}  // namespace

}  // namespace motif

extern "C" int motif_probe_copy(const void *src, void *dst, size_t bytes, int grid, void *stream) {
  using namespace motif;
  if (!src || !dst || bytes % 16 || grid <= 0) return set_error(MOTIF_ERR_INVALID, "probe_copy: bad arguments");
  probe_copy_kernel<<<dim3(grid), dim3(kProbeThreads), 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint4 *>(src), static_cast<uint4 *>(dst), bytes / 16);
  return check_launch("probe_copy_kernel");
}

extern "C" int motif_probe_read(const void *src, void *out, size_t bytes, int grid, void *stream) {
  using namespace motif;
  if (!src || !out || bytes % 16 || grid <= 0) return set_error(MOTIF_ERR_INVALID, "probe_read: bad arguments");
  probe_read_kernel<<<dim3(grid), dim3(kProbeThreads), 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint4 *>(src), static_cast<uint32_t *>(out), bytes / 16);
  return check_launch("probe_read_kernel");
}

extern "C" int motif_probe_mfma_bf16(void *out, int grid, int iters, int shape, void *stream) {
  using namespace motif;
  if (!out || grid <= 0 || iters <= 0 || (shape != 16 && shape != 32))
    return set_error(MOTIF_ERR_INVALID, "probe_mfma: bad arguments");
  if (shape == 32) {
    probe_mfma32_kernel<<<dim3(grid), dim3(kProbeThreads), 0, static_cast<hipStream_t>(stream)>>>(
        static_cast<float *>(out), iters, 1e-3f);
    return check_launch("probe_mfma32_kernel");
  }
  probe_mfma_kernel<<<dim3(grid), dim3(kProbeThreads), 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<float *>(out), iters, 1e-3f);
  return check_launch("probe_mfma_kernel");
}

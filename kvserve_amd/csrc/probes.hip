// Measurement probes (no counterpart in the reference; bench.py --probes): what this GPU
// sustains for the two resources the attention kernels are bound by, measured with the same
// access widths the kernels use, so a kernel's rate can be read against an attainable ceiling
// as well as against the published peak.
//
//  * stream read: 16-byte loads per lane (ordinary, or non-temporal as the decode kernels'
//    K/V loads), each workgroup reading its own contiguous range of a buffer much larger than
//    the Infinity Cache, kProbeUnroll loads in flight per thread (32 KB per workgroup), an XOR
//    of everything read kept per thread (so no load is dead) and one dword written per thread:
//    the HBM read rate a streaming kernel can reach. (A grid-stride walk, where consecutive
//    loads of a thread lie a whole grid apart, read 8-10% slower.)
//  * page gather: the decode kernels' access pattern: 4 KB pages in a scattered order (page
//    j of the walk is page (j * 0x9E3779B1) mod npages, a bijection for a power-of-two
//    count), each wave taking its own run of the walk with kGatherPages pages (16 loads of
//    16 bytes per lane) in flight, non-temporal loads, XOR kept as above: the read rate the
//    decode kernels' bound is measured against.
//  * copy: the same loads, each vector stored to a second buffer: read + write rate (the cache
//    write's bound).
//  * mfma: each wave runs kProbeChains independent accumulator chains of
//    v_mfma_f32_16x16x32_bf16 (the prefill kernel's instruction) for `iters` steps, operands in
//    registers; the dense bf16 rate the matrix cores sustain.
//  * co-issue: an MFMA wave and a softmax-like VALU wave on each SIMD, and one wave interleaving
//    its own independent FMAs between MFMAs (below).
#include "kvh_device.h"
#include "kvh_internal.h"

namespace kvh {

constexpr int kProbeUnroll = 8;
constexpr int kProbeChains = 4;

// NT: non-temporal loads (the decode kernels' K/V loads), else ordinary ones
template <bool NT>
__device__ __forceinline__ u32x4 probe_load(const u32x4* p) {
  if constexpr (NT)
    return __builtin_nontemporal_load(p);
  else
    return *p;
}

// workgroup b reads 16-byte elements [n b / blocks, n (b + 1) / blocks)
template <bool NT>
__global__ __launch_bounds__(256) void probe_stream_read_kernel(const u32x4* src, int64_t n, uint32_t* sink) {
  const int64_t lo = n * blockIdx.x / gridDim.x, hi = n * (blockIdx.x + 1) / gridDim.x;
  int64_t i = lo + threadIdx.x;
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (; i + (kProbeUnroll - 1) * 256 < hi; i += kProbeUnroll * 256) {
    u32x4 v[kProbeUnroll];
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) v[u] = probe_load<NT>(src + i + u * 256);
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) acc ^= v[u];
  }
  for (; i < hi; i += 256) acc ^= probe_load<NT>(src + i);
  sink[(int64_t)blockIdx.x * 256 + threadIdx.x] = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
}

constexpr int kGatherPages = 4;
constexpr int kPage16 = 256;  // 16-byte elements per 4 KB page

// npages a power of two; wave w of the grid walks positions [npages w / W, npages (w + 1) / W)
__global__ __launch_bounds__(256) void probe_page_gather_kernel(const u32x4* src, int64_t npages, uint32_t* sink) {
  const int64_t waves = (int64_t)gridDim.x * 4;
  const int64_t w = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int64_t lo = npages * w / waves, hi = npages * (w + 1) / waves;
  auto page = [&](int64_t j) { return src + (int64_t)(((uint64_t)j * 0x9E3779B1ull) & (uint64_t)(npages - 1)) * kPage16 + lane; };
  u32x4 acc = {0u, 0u, 0u, 0u};
  int64_t j = lo;
  for (; j + kGatherPages <= hi; j += kGatherPages) {
    u32x4 v[kGatherPages][4];
#pragma unroll
    for (int q = 0; q < kGatherPages; ++q) {
      const u32x4* pg = page(j + q);
#pragma unroll
      for (int c = 0; c < 4; ++c) v[q][c] = probe_load<true>(pg + 64 * c);
    }
#pragma unroll
    for (int q = 0; q < kGatherPages; ++q)
#pragma unroll
      for (int c = 0; c < 4; ++c) acc ^= v[q][c];
  }
  for (; j < hi; ++j) {
    const u32x4* pg = page(j);
#pragma unroll
    for (int c = 0; c < 4; ++c) acc ^= probe_load<true>(pg + 64 * c);
  }
  sink[(int64_t)blockIdx.x * 256 + threadIdx.x] = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
}

// the same ranges as the stream read
__global__ __launch_bounds__(256) void probe_copy_kernel(const u32x4* src, u32x4* dst, int64_t n) {
  const int64_t lo = n * blockIdx.x / gridDim.x, hi = n * (blockIdx.x + 1) / gridDim.x;
  int64_t i = lo + threadIdx.x;
  for (; i + (kProbeUnroll - 1) * 256 < hi; i += kProbeUnroll * 256) {
    u32x4 v[kProbeUnroll];
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) v[u] = src[i + u * 256];
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) dst[i + u * 256] = v[u];
  }
  for (; i < hi; i += 256) dst[i] = src[i];
}

__global__ __launch_bounds__(256) void probe_mfma_kernel(int iters, float* sink) {
  const uint32_t lane = threadIdx.x & 63;
  // operands that differ by lane and wave (nothing folds), bf16 values near 1
  const uint32_t x = 0x3f803f80u ^ ((lane * 0x00010001u + blockIdx.x) & 0x000f000fu);
  const u32x4 a = {x, x ^ 1u, x ^ 2u, x ^ 3u}, b = {x ^ 4u, x ^ 5u, x ^ 6u, x ^ 7u};
  f32x4 c[kProbeChains];
#pragma unroll
  for (int k = 0; k < kProbeChains; ++k) c[k] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int k = 0; k < kProbeChains; ++k) c[k] = BF16::mfma(a, b, c[k]);
  }
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < kProbeChains; ++k) s += c[k][0] + c[k][1] + c[k][2] + c[k][3];
  sink[(int64_t)blockIdx.x * 256 + threadIdx.x] = s;
}

// Co-issue on one SIMD: 512-thread workgroups, one per CU; waves 0-3 (one per SIMD) run
// iters_m steps of kProbeChains MFMA chains, waves 4-7 (the second wave of each SIMD) run
// iters_v steps of a softmax's vector work per 16 scores (16 FMA + 16 exp2, 8 packs to bf16 and
// 8 dot2 row-sum steps); either count 0 leaves those waves idle. Timed three ways it shows how
// much of the VALU time hides under the MFMAs of the other wave.
__global__ __launch_bounds__(512, 1) void probe_coissue_kernel(int iters_m, int iters_v, float* sink) {
  const int w = threadIdx.x >> 6;
  float s = 0.f;
  if (w < 4) {
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t x = 0x3f803f80u ^ ((lane * 0x00010001u + blockIdx.x) & 0x000f000fu);
    const u32x4 a = {x, x ^ 1u, x ^ 2u, x ^ 3u}, b = {x ^ 4u, x ^ 5u, x ^ 6u, x ^ 7u};
    f32x4 c[kProbeChains];
#pragma unroll
    for (int k = 0; k < kProbeChains; ++k) c[k] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int it = 0; it < iters_m; ++it) {
#pragma unroll
      for (int k = 0; k < kProbeChains; ++k) c[k] = BF16::mfma(a, b, c[k]);
    }
#pragma unroll
    for (int k = 0; k < kProbeChains; ++k) s += c[k][0] + c[k][3];
  } else {
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) x[i] = -0.01f * (float)((threadIdx.x + i) & 63);
    float l = 0.f;
    for (int it = 0; it < iters_v; ++it) {
      float pv[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) pv[i] = fast_exp2(__builtin_fmaf(x[i], 0.7f, -0.3f));
#pragma unroll
      for (int i = 0; i < 16; i += 2) {
        const uint32_t pk = BF16::pack2(pv[i], pv[i + 1]);
        l = BF16::dot2_ones(pk, l);
        x[i] = -pv[i + 1];
        x[i + 1] = -pv[i];
      }
    }
    s = l + x[0];
  }
  sink[(int64_t)blockIdx.x * 512 + threadIdx.x] = s;
}

// Co-issue within one wave: waves of 256-thread workgroups run iters steps of 8 MFMA chains,
// each MFMA followed by NV independent FMAs (sched_group_barrier keeps them interleaved); timed
// against NV = 0, the VALU time the MFMAs do not hide.
template <int NV>
__global__ __launch_bounds__(256) void probe_interleave_kernel(int iters, float* sink) {
  constexpr int NC = 8;
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t x0 = 0x3f803f80u ^ ((lane * 0x00010001u + blockIdx.x) & 0x000f000fu);
  const u32x4 a = {x0, x0 ^ 1u, x0 ^ 2u, x0 ^ 3u}, b = {x0 ^ 4u, x0 ^ 5u, x0 ^ 6u, x0 ^ 7u};
  f32x4 c[NC];
#pragma unroll
  for (int k = 0; k < NC; ++k) c[k] = f32x4{0.f, 0.f, 0.f, 0.f};
  float x[NV > 0 ? NV : 1];
#pragma unroll
  for (int i = 0; i < (NV > 0 ? NV : 1); ++i) x[i] = 0.01f * (float)(lane + i);
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int k = 0; k < NC; ++k) {
      c[k] = BF16::mfma(a, b, c[k]);
#pragma unroll
      for (int i = 0; i < NV; ++i) x[i] = __builtin_fmaf(x[i], 0.999f, 0.001f);
    }
    if constexpr (NV > 0) {
#pragma unroll
      for (int k = 0; k < NC; ++k) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, NV, 0);
      }
    }
  }
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < NC; ++k) s += c[k][0] + c[k][3];
#pragma unroll
  for (int i = 0; i < (NV > 0 ? NV : 1); ++i) s += x[i];
  sink[(int64_t)blockIdx.x * 256 + threadIdx.x] = s;
}

int launch_probe(int kind, const void* src, void* dst, int64_t bytes, int32_t blocks, int32_t iters,
                 hipStream_t s) {
  if (kind == 4) {
    float* sink = (float*)dst;
    switch ((int)bytes) {
      case 0: hipLaunchKernelGGL(probe_interleave_kernel<0>, dim3(blocks), dim3(256), 0, s, iters, sink); break;
      case 1: hipLaunchKernelGGL(probe_interleave_kernel<1>, dim3(blocks), dim3(256), 0, s, iters, sink); break;
      case 2: hipLaunchKernelGGL(probe_interleave_kernel<2>, dim3(blocks), dim3(256), 0, s, iters, sink); break;
      case 3: hipLaunchKernelGGL(probe_interleave_kernel<3>, dim3(blocks), dim3(256), 0, s, iters, sink); break;
      default: hipLaunchKernelGGL(probe_interleave_kernel<4>, dim3(blocks), dim3(256), 0, s, iters, sink); break;
    }
    return (int)hipGetLastError();
  }
  if (kind == 3) {
    hipLaunchKernelGGL(probe_coissue_kernel, dim3(blocks), dim3(512), 0, s, iters, (int)bytes, (float*)dst);
    return (int)hipGetLastError();
  }
  const int64_t n = bytes / 16;
  if (kind == 0)
    hipLaunchKernelGGL(probe_stream_read_kernel<false>, dim3(blocks), dim3(256), 0, s, (const u32x4*)src, n,
                       (uint32_t*)dst);
  else if (kind == 5)
    hipLaunchKernelGGL(probe_stream_read_kernel<true>, dim3(blocks), dim3(256), 0, s, (const u32x4*)src, n,
                       (uint32_t*)dst);
  else if (kind == 6)
    hipLaunchKernelGGL(probe_page_gather_kernel, dim3(blocks), dim3(256), 0, s, (const u32x4*)src, n / kPage16,
                       (uint32_t*)dst);
  else if (kind == 1)
    hipLaunchKernelGGL(probe_copy_kernel, dim3(blocks), dim3(256), 0, s, (const u32x4*)src, (u32x4*)dst, n);
  else
    hipLaunchKernelGGL(probe_mfma_kernel, dim3(blocks), dim3(256), 0, s, iters, (float*)dst);
  return (int)hipGetLastError();
}

}  // namespace kvh

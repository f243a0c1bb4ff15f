// Engine-harness kernels around the attention path: the elementwise steps of a Llama layer
// fused into single passes, and a weight-streaming GEMV for decode-sized batches. They serve
// kvserve_amd.engine (the counterpart of the reference's model.py), not the attention ABI.
//
//   add_rmsnorm: x' = x + delta (rounded to the storage type, as PyTorch's add), then
//                h = weight * (x' * rsqrt(mean(x'^2) + eps)).to(dtype)   (model.py:22-32)
//                one workgroup per token row; replaces an add and seven norm kernels.
//   silu_mul:    out = silu(gate).to(dtype) * up (model.py MLP), gate / up the two halves of
//                the fused gate_up projection; replaces a chunk view, silu and a multiply.
//   gemv:        y[m][n] = sum_k x[m][k] w[n][k] for m < M <= 8 (nn.Linear with a [N, K]
//                weight), fp32 accumulation; HBM-bound on the weight, which each wave
//                streams in 1 KB loads while x comes from L1/L2.
//   gemv + silu_mul (GLU): the gate_up projection with silu_mul in its epilogue: a wave
//                takes gate rows j .. and the up rows I + j .., rounds both sums to the
//                storage type (the projection's output) and applies silu_mul's arithmetic.
#include "kvh_device.h"
#include "kvh_internal.h"

namespace kvh {
namespace {

constexpr int kOpsThreads = 256;

template <class E>
__device__ __forceinline__ void unpack8(const u32x4& w, float (&f)[8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) f[i] = E::to_f32((uint16_t)(w[i / 2] >> (16 * (i & 1))));
}

template <class E>
__device__ __forceinline__ u32x4 pack8(const float (&f)[8]) {
  return u32x4{E::pack2(f[0], f[1]), E::pack2(f[2], f[3]), E::pack2(f[4], f[5]), E::pack2(f[6], f[7])};
}

__device__ __forceinline__ float block_sum(float v, float* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < kOpsThreads / 64; ++i) s += red[i];
  return s;
}

// A thread keeps its first kKeep vectors (hd <= 8192) and their norm weights in registers
// between the two passes, so the second pass starts without a memory round trip; wider rows
// re-read the rest.
constexpr int kKeep = 4;

template <class E>
__global__ __launch_bounds__(kOpsThreads) void add_rmsnorm_kernel(const uint16_t* __restrict__ x, int64_t x_ts,
                                                                  const uint16_t* __restrict__ d, int64_t d_ts,
                                                                  const uint16_t* __restrict__ w,
                                                                  uint16_t* __restrict__ xo, int64_t xo_ts,
                                                                  uint16_t* __restrict__ h, int64_t h_ts, int hd,
                                                                  float eps) {
  __shared__ float red[kOpsThreads / 64];
  const int64_t t = blockIdx.x;
  const int nv = hd / 8;
  const uint16_t* xr = x + t * x_ts;
  uint16_t* xor_ = xo + t * xo_ts;
  float keep[kKeep][8];
  u32x4 wkeep[kKeep];
  float ss = 0.f;
  auto sum_in = [&](int v, float (&a)[8]) {
    unpack8<E>(*(const u32x4*)(xr + 8 * v), a);
    if (d) {
      float b[8];
      unpack8<E>(*(const u32x4*)(d + t * d_ts + 8 * v), b);
#pragma unroll
      for (int i = 0; i < 8; ++i) a[i] += b[i];
      const u32x4 o = pack8<E>(a);
      *(u32x4*)(xor_ + 8 * v) = o;
      unpack8<E>(o, a);  // the rounded sum is what the norm sees
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) ss = __builtin_fmaf(a[i], a[i], ss);
  };
#pragma unroll
  for (int j = 0; j < kKeep; ++j) {
    const int v = threadIdx.x + kOpsThreads * j;
    if (v < nv) {
      wkeep[j] = *(const u32x4*)(w + 8 * v);
      sum_in(v, keep[j]);
    }
  }
  for (int v = threadIdx.x + kOpsThreads * kKeep; v < nv; v += kOpsThreads) {
    float a[8];
    sum_in(v, a);
  }
  const float r = rsqrtf(block_sum(ss, red) / (float)hd + eps);
  auto norm_out = [&](int v, float (&a)[8], const u32x4& wv) {
    float g[8];
    unpack8<E>(wv, g);
#pragma unroll
    for (int i = 0; i < 8; ++i) a[i] *= r;
    unpack8<E>(pack8<E>(a), a);  // .to(dtype) before the weight
#pragma unroll
    for (int i = 0; i < 8; ++i) a[i] *= g[i];
    *(u32x4*)(h + t * h_ts + 8 * v) = pack8<E>(a);
  };
#pragma unroll
  for (int j = 0; j < kKeep; ++j) {
    const int v = threadIdx.x + kOpsThreads * j;
    if (v < nv) norm_out(v, keep[j], wkeep[j]);
  }
  const uint16_t* src = d ? xor_ : xr;
  for (int v = threadIdx.x + kOpsThreads * kKeep; v < nv; v += kOpsThreads) {
    float a[8];
    unpack8<E>(*(const u32x4*)(src + 8 * v), a);
    norm_out(v, a, *(const u32x4*)(w + 8 * v));
  }
}

template <class E>
__global__ __launch_bounds__(kOpsThreads) void silu_mul_kernel(const uint16_t* __restrict__ gu, int64_t gu_ts,
                                                               uint16_t* __restrict__ out, int64_t o_ts, int inter) {
  const int64_t t = blockIdx.y;
  const int v = blockIdx.x * kOpsThreads + threadIdx.x;
  if (8 * v >= inter) return;
  float g[8], u[8];
  unpack8<E>(*(const u32x4*)(gu + t * gu_ts + 8 * v), g);
  unpack8<E>(*(const u32x4*)(gu + t * gu_ts + inter + 8 * v), u);
#pragma unroll
  for (int i = 0; i < 8; ++i) g[i] = g[i] / (1.f + expf(-g[i]));
  unpack8<E>(pack8<E>(g), g);  // silu(gate) in the storage type, then the product
#pragma unroll
  for (int i = 0; i < 8; ++i) g[i] *= u[i];
  *(u32x4*)(out + t * o_ts + 8 * v) = pack8<E>(g);
}

// GEMV: a wave owns RW consecutive weight rows and walks k in steps of 512 (64 lanes x 8
// elements, one 16-byte load per lane per row), two steps per iteration so 2 RW weight loads
// are in flight; lane partial sums are reduced across the wave at the end. Products are
// accumulated with explicit FMAs (no two-product dot instructions), so a row's sum has the
// same bits in every instantiation.
// silu_mul of one (gate, up) pair of fp32 sums, each first rounded to the storage type
template <class E>
__device__ __forceinline__ float silu_mul1(float g, float u) {
  g = E::to_f32((uint16_t)(E::pack2(g, 0.f) & 0xffffu));
  u = E::to_f32((uint16_t)(E::pack2(u, 0.f) & 0xffffu));
  g = g / (1.f + expf(-g));
  g = E::to_f32((uint16_t)(E::pack2(g, 0.f) & 0xffffu));
  return g * u;
}

// GLU: n is the intermediate size I; the weight has 2 I rows (gate, then up); wave rows
// r < RW / 2 are gate rows n0 + r, the others up rows I + n0 + r - RW / 2, n0 = wave RW / 2.
template <class E, int M, int RW, bool GLU = false>
__global__ __launch_bounds__(kOpsThreads) void gemv_kernel(const uint16_t* __restrict__ x, int64_t x_rs,
                                                           const uint16_t* __restrict__ w, int64_t w_rs,
                                                           uint16_t* __restrict__ y, int64_t y_rs, int n, int k) {
  constexpr int OUT = GLU ? RW / 2 : RW;  // outputs per wave
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * (kOpsThreads / 64) + (threadIdx.x >> 6);
  const int n0 = wave * OUT;
  if (n0 >= n) return;
  float acc[M][RW];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < RW; ++r) acc[m][r] = 0.f;
  const uint16_t* wr[RW];
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    if constexpr (GLU)  // rows past n repeat the last gate / up row
      wr[r] = w + ((int64_t)(r < OUT ? 0 : n) + min(n0 + r % OUT, n - 1)) * w_rs;
    else
      wr[r] = w + (int64_t)min(n0 + r, n - 1) * w_rs;  // rows past n repeat the last
  }
  const int kfull = k / 1024 * 1024;
  for (int k0 = 8 * lane; k0 < kfull; k0 += 1024) {
    u32x4 wv[2][RW], xv[2][M];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
#pragma unroll
      for (int r = 0; r < RW; ++r) wv[s][r] = *(const u32x4*)(wr[r] + k0 + 512 * s);
#pragma unroll
      for (int m = 0; m < M; ++m) xv[s][m] = *(const u32x4*)(x + m * x_rs + k0 + 512 * s);
    }
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int m = 0; m < M; ++m) {
        float xf[8];
        unpack8<E>(xv[s][m], xf);
#pragma unroll
        for (int r = 0; r < RW; ++r) {
          float wf[8];
          unpack8<E>(wv[s][r], wf);
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[m][r] = __builtin_fmaf(xf[i], wf[i], acc[m][r]);
        }
      }
  }
  for (int k0 = kfull + 8 * lane; k0 < k; k0 += 512) {  // tail: k % 1024 (k % 8 == 0)
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float xf[8];
      unpack8<E>(*(const u32x4*)(x + m * x_rs + k0), xf);
#pragma unroll
      for (int r = 0; r < RW; ++r) {
        float wf[8];
        unpack8<E>(*(const u32x4*)(wr[r] + k0), wf);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[m][r] = __builtin_fmaf(xf[i], wf[i], acc[m][r]);
      }
    }
  }
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      float v = acc[m][r];
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
      acc[m][r] = v;
    }
  if (lane == 0) {
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
      for (int r = 0; r < OUT; ++r) {
        if (n0 + r >= n) continue;
        const float v = GLU ? silu_mul1<E>(acc[m][r], acc[m][r + OUT]) : acc[m][r];
        y[m * y_rs + n0 + r] = (uint16_t)(E::pack2(v, 0.f) & 0xffffu);
      }
  }
}

template <class E, int M>
int launch_gemv_m(const void* x, int64_t x_rs, const void* w, int64_t w_rs, void* y, int64_t y_rs, int n, int k,
                  hipStream_t s) {
  // rows per wave: enough waves to fill the chip for small n, fewer reductions for large n
  const int rw = n >= 16384 ? 4 : (n >= 4096 ? 2 : 1);
  const int waves = (n + rw - 1) / rw;
  const dim3 grid((waves + kOpsThreads / 64 - 1) / (kOpsThreads / 64));
  if (rw == 4)
    hipLaunchKernelGGL((gemv_kernel<E, M, 4>), grid, dim3(kOpsThreads), 0, s, (const uint16_t*)x, x_rs,
                       (const uint16_t*)w, w_rs, (uint16_t*)y, y_rs, n, k);
  else if (rw == 2)
    hipLaunchKernelGGL((gemv_kernel<E, M, 2>), grid, dim3(kOpsThreads), 0, s, (const uint16_t*)x, x_rs,
                       (const uint16_t*)w, w_rs, (uint16_t*)y, y_rs, n, k);
  else
    hipLaunchKernelGGL((gemv_kernel<E, M, 1>), grid, dim3(kOpsThreads), 0, s, (const uint16_t*)x, x_rs,
                       (const uint16_t*)w, w_rs, (uint16_t*)y, y_rs, n, k);
  return (int)hipGetLastError();
}

// gate_up + silu_mul: two gate and two up rows per wave (4 weight rows in flight)
template <class E, int M>
int launch_gemv_glu_m(const void* x, int64_t x_rs, const void* w, int64_t w_rs, void* y, int64_t y_rs, int inter,
                      int k, hipStream_t s) {
  const int waves = (inter + 1) / 2;
  const dim3 grid((waves + kOpsThreads / 64 - 1) / (kOpsThreads / 64));
  hipLaunchKernelGGL((gemv_kernel<E, M, 4, true>), grid, dim3(kOpsThreads), 0, s, (const uint16_t*)x, x_rs,
                     (const uint16_t*)w, w_rs, (uint16_t*)y, y_rs, inter, k);
  return (int)hipGetLastError();
}

template <class E>
int launch_gemv_glu_t(const void* x, int64_t x_rs, const void* w, int64_t w_rs, void* y, int64_t y_rs, int m,
                      int inter, int k, hipStream_t s) {
  switch (m) {
    case 1: return launch_gemv_glu_m<E, 1>(x, x_rs, w, w_rs, y, y_rs, inter, k, s);
    case 2: return launch_gemv_glu_m<E, 2>(x, x_rs, w, w_rs, y, y_rs, inter, k, s);
    case 3: return launch_gemv_glu_m<E, 3>(x, x_rs, w, w_rs, y, y_rs, inter, k, s);
    default: return launch_gemv_glu_m<E, 4>(x, x_rs, w, w_rs, y, y_rs, inter, k, s);
  }
}

template <class E>
int launch_gemv_t(const void* x, int64_t x_rs, const void* w, int64_t w_rs, void* y, int64_t y_rs, int m, int n,
                  int k, hipStream_t s) {
  switch (m) {
    case 1: return launch_gemv_m<E, 1>(x, x_rs, w, w_rs, y, y_rs, n, k, s);
    case 2: return launch_gemv_m<E, 2>(x, x_rs, w, w_rs, y, y_rs, n, k, s);
    case 3: return launch_gemv_m<E, 3>(x, x_rs, w, w_rs, y, y_rs, n, k, s);
    case 4: return launch_gemv_m<E, 4>(x, x_rs, w, w_rs, y, y_rs, n, k, s);
    case 5: return launch_gemv_m<E, 5>(x, x_rs, w, w_rs, y, y_rs, n, k, s);
    case 6: return launch_gemv_m<E, 6>(x, x_rs, w, w_rs, y, y_rs, n, k, s);
    case 7: return launch_gemv_m<E, 7>(x, x_rs, w, w_rs, y, y_rs, n, k, s);
    default: return launch_gemv_m<E, 8>(x, x_rs, w, w_rs, y, y_rs, n, k, s);
  }
}

// Skinny GEMM for 5 .. 64 rows: y[m][n] = sum_k x[m][k] w[n][k] on v_mfma_f32_16x16x32. A
// workgroup of 8 waves owns 16 weight rows (one MFMA A tile, n0 .. n0 + 15); wave w takes the
// k-slice [w K / 8, (w + 1) K / 8) in 32-wide steps, four in flight, with MT = ceil(m / 16)
// B tiles of x (rows past m read row m - 1 and are dropped). The 8 partial 16 x 16 MT tiles
// meet in LDS and are summed in wave order (deterministic) and rounded once. Lane l of a tile
// holds D[4 (l / 16) + r][l % 16], r < 4: weight row n0 + 4 (l / 16) + r, x row 16 mt + l % 16.
// GLU: the workgroup owns output columns c0 .. c0 + 7 (c0 = 8 blockIdx) of silu_mul(gate_up):
// A rows i < 8 are gate rows c0 + i, rows i >= 8 the up rows inter + c0 + i - 8; the epilogue
// rounds each sum to the storage type and applies silu_mul's arithmetic (the bits of the plain
// kernel followed by kvh_silu_mul). n is then the intermediate size.
constexpr int kSkinnyWaves = 8;

template <class E, int MT, bool GLU = false>
__global__ __launch_bounds__(64 * kSkinnyWaves) void skinny_gemm_kernel(const uint16_t* __restrict__ x,
                                                                        int64_t x_rs,
                                                                        const uint16_t* __restrict__ w,
                                                                        int64_t w_rs, uint16_t* __restrict__ y,
                                                                        int64_t y_rs, int m, int k, int n) {
  __shared__ f32x4 red[kSkinnyWaves][MT][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int i = lane & 15, j = lane >> 4;
  const int64_t n0 = (int64_t)blockIdx.x * (GLU ? 8 : 16);
  const int slice = k / kSkinnyWaves;
  const int k_lo = wave * slice;
  const int64_t wrow = GLU ? (i < 8 ? n0 + i : n + n0 + i - 8) : n0 + i;
  const uint16_t* wr = w + wrow * w_rs + k_lo + 8 * j;
  const uint16_t* xr[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) xr[t] = x + (int64_t)min(16 * t + i, m - 1) * x_rs + k_lo + 8 * j;
  f32x4 acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int kk = 0; kk < slice; kk += 128) {
    u32x4 a[4], b[4][MT];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      a[u] = *(const u32x4*)(wr + kk + 32 * u);
#pragma unroll
      for (int t = 0; t < MT; ++t) b[u][t] = *(const u32x4*)(xr[t] + kk + 32 * u);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int t = 0; t < MT; ++t) acc[t] = E::mfma(a[u], b[u][t], acc[t]);
  }
#pragma unroll
  for (int t = 0; t < MT; ++t) red[wave][t][lane] = acc[t];
  __syncthreads();
  if constexpr (GLU) {
    // 8 x 16 MT outputs; thread q: column c = q % 8 of x row 16 t + (q / 8) % 16, t = q / 128;
    // the gate sum is D[c][.] (lane 16 (c / 4) + row, element c % 4), the up sum D[8 + c][.]
    for (int q = threadIdx.x; q < MT * 128; q += 64 * kSkinnyWaves) {
      const int t = q >> 7, mr = (q >> 3) & 15, c = q & 7;
      const int row = 16 * t + mr;
      if (row >= m) continue;
      const int lg = 16 * (c >> 2) + mr, lu = 16 * (2 + (c >> 2)) + mr, r = c & 3;
      float g = 0.f, u = 0.f;
#pragma unroll
      for (int v = 0; v < kSkinnyWaves; ++v) {
        g += red[v][t][lg][r];
        u += red[v][t][lu][r];
      }
      y[row * y_rs + n0 + c] = (uint16_t)(E::pack2(silu_mul1<E>(g, u), 0.f) & 0xffffu);
    }
  } else {
    // 16 x 16 MT outputs; thread q sums element q % 4 of lane (q / 4) % 64 of tile q / 256
    for (int q = threadIdx.x; q < MT * 256; q += 64 * kSkinnyWaves) {
      const int t = q >> 8, l = (q >> 2) & 63, r = q & 3;
      const int row = 16 * t + (l & 15);
      if (row >= m) continue;
      float sum = 0.f;
#pragma unroll
      for (int v = 0; v < kSkinnyWaves; ++v) sum += red[v][t][l][r];
      y[row * y_rs + n0 + 4 * (l >> 4) + r] = (uint16_t)(E::pack2(sum, 0.f) & 0xffffu);
    }
  }
}

template <class E, bool GLU>
int launch_skinny_t(const void* x, int64_t x_rs, const void* w, int64_t w_rs, void* y, int64_t y_rs, int m, int n,
                    int k, hipStream_t s) {
  const dim3 grid((unsigned)(n / (GLU ? 8 : 16))), block(64 * kSkinnyWaves);
  const auto* xp = (const uint16_t*)x;
  const auto* wp = (const uint16_t*)w;
  auto* yp = (uint16_t*)y;
  switch ((m + 15) / 16) {
    case 1: hipLaunchKernelGGL((skinny_gemm_kernel<E, 1, GLU>), grid, block, 0, s, xp, x_rs, wp, w_rs, yp, y_rs, m, k, n); break;
    case 2: hipLaunchKernelGGL((skinny_gemm_kernel<E, 2, GLU>), grid, block, 0, s, xp, x_rs, wp, w_rs, yp, y_rs, m, k, n); break;
    case 3: hipLaunchKernelGGL((skinny_gemm_kernel<E, 3, GLU>), grid, block, 0, s, xp, x_rs, wp, w_rs, yp, y_rs, m, k, n); break;
    default: hipLaunchKernelGGL((skinny_gemm_kernel<E, 4, GLU>), grid, block, 0, s, xp, x_rs, wp, w_rs, yp, y_rs, m, k, n); break;
  }
  return (int)hipGetLastError();
}

}  // namespace

int launch_add_rmsnorm(const void* x, int64_t x_ts, const void* d, int64_t d_ts, const void* w, void* xo,
                       int64_t xo_ts, void* h, int64_t h_ts, int64_t T, int32_t hd, float eps, int32_t dtype,
                       hipStream_t s) {
  if (T == 0) return 0;
  if (dtype == 2)
    hipLaunchKernelGGL((add_rmsnorm_kernel<BF16>), dim3((unsigned)T), dim3(kOpsThreads), 0, s, (const uint16_t*)x,
                       x_ts, (const uint16_t*)d, d_ts, (const uint16_t*)w, (uint16_t*)xo, xo_ts, (uint16_t*)h, h_ts,
                       hd, eps);
  else
    hipLaunchKernelGGL((add_rmsnorm_kernel<F16>), dim3((unsigned)T), dim3(kOpsThreads), 0, s, (const uint16_t*)x,
                       x_ts, (const uint16_t*)d, d_ts, (const uint16_t*)w, (uint16_t*)xo, xo_ts, (uint16_t*)h, h_ts,
                       hd, eps);
  return (int)hipGetLastError();
}

int launch_silu_mul(const void* gu, int64_t gu_ts, void* out, int64_t o_ts, int64_t T, int32_t inter, int32_t dtype,
                    hipStream_t s) {
  if (T == 0) return 0;
  const dim3 grid((unsigned)((inter / 8 + kOpsThreads - 1) / kOpsThreads), (unsigned)T);
  if (dtype == 2)
    hipLaunchKernelGGL((silu_mul_kernel<BF16>), grid, dim3(kOpsThreads), 0, s, (const uint16_t*)gu, gu_ts,
                       (uint16_t*)out, o_ts, inter);
  else
    hipLaunchKernelGGL((silu_mul_kernel<F16>), grid, dim3(kOpsThreads), 0, s, (const uint16_t*)gu, gu_ts,
                       (uint16_t*)out, o_ts, inter);
  return (int)hipGetLastError();
}

int launch_gemv(const void* x, int64_t x_rs, const void* w, int64_t w_rs, void* y, int64_t y_rs, int32_t m, int32_t n,
                int32_t k, int32_t dtype, hipStream_t s) {
  return dtype == 2 ? launch_gemv_t<BF16>(x, x_rs, w, w_rs, y, y_rs, m, n, k, s)
                    : launch_gemv_t<F16>(x, x_rs, w, w_rs, y, y_rs, m, n, k, s);
}

int launch_gemv_silu_mul(const void* x, int64_t x_rs, const void* w, int64_t w_rs, void* y, int64_t y_rs, int32_t m,
                         int32_t inter, int32_t k, int32_t dtype, hipStream_t s) {
  return dtype == 2 ? launch_gemv_glu_t<BF16>(x, x_rs, w, w_rs, y, y_rs, m, inter, k, s)
                    : launch_gemv_glu_t<F16>(x, x_rs, w, w_rs, y, y_rs, m, inter, k, s);
}

int launch_gemm_skinny(const void* x, int64_t x_rs, const void* w, int64_t w_rs, void* y, int64_t y_rs, int32_t m,
                       int32_t n, int32_t k, bool glu, int32_t dtype, hipStream_t s) {
  if (glu)
    return dtype == 2 ? launch_skinny_t<BF16, true>(x, x_rs, w, w_rs, y, y_rs, m, n, k, s)
                      : launch_skinny_t<F16, true>(x, x_rs, w, w_rs, y, y_rs, m, n, k, s);
  return dtype == 2 ? launch_skinny_t<BF16, false>(x, x_rs, w, w_rs, y, y_rs, m, n, k, s)
                    : launch_skinny_t<F16, false>(x, x_rs, w, w_rs, y, y_rs, m, n, k, s);
}

}  // namespace kvh

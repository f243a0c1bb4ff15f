// Exact-fp32 paged attention (the reference's IEEE mode, src/kvserve/kernels/paged_attention.py:92-95,
// :106-109, used by its fp32 engine identity tests). Correctness path, not a bandwidth path:
// plain fp32 FMA on the vector ALUs, any head_dim <= 256 (multiple of 4) and any block size.
//
// Grid (B, H, ceil(max_q / kRowsPerWG)); one wave per workgroup walks the query tokens
// q0, q0 + 1, ... of its (sequence, head) one at a time. For each 64-key tile, lane k scores
// key k (full dot product over d), the wave does an online-softmax update, then every lane
// accumulates its own d columns over the tile's keys.
#include "kvh_device.h"
#include "kvh_internal.h"

namespace kvh {

constexpr int kRowsPerWG = 8;

template <int DPL>  // d columns per lane: d = lane + 64 * x, x < DPL
__global__ __launch_bounds__(64) void pa_f32_kernel(PAParams p, int D) {
  const int seq = blockIdx.x, head = blockIdx.y;
  const int lane = threadIdx.x;
  const int kvh = head / p.G;
  const int64_t qs = clamp64(p.qsl[seq], 0, p.T);
  const int64_t qe = clamp64(p.qsl[seq + 1], qs, p.T);
  const int q_len = (int)(qe - qs);
  const int64_t sl = p.seq_lens[seq];
  const int64_t ctx = sl - q_len;
  const int kv_total = (int)clamp64(sl, 0, (int64_t)p.W * p.BS);
  const int64_t* btrow = p.bt + (int64_t)seq * p.bt_rs;
  const float* kc = (const float*)p.kc;
  const float* vc = (const float*)p.vc;
  __shared__ float s_q[256];

  const int qi_end = min(q_len, (int)(blockIdx.z + 1) * kRowsPerWG);
  for (int qi = blockIdx.z * kRowsPerWG; qi < qi_end; ++qi) {
    const int64_t tok = qs + qi;
    const float* qrow = (const float*)p.q + tok * p.q_ts + (int64_t)head * p.q_hs;
    __syncthreads();
    for (int d = lane; d < D; d += 64) s_q[d] = qrow[d];
    __syncthreads();
    const int limit = (int)clamp64(ctx + qi + 1, 0, kv_total);
    float m = -INFINITY, l = 0.f;
    float acc[DPL];
#pragma unroll
    for (int x = 0; x < DPL; ++x) acc[x] = 0.f;

    for (int k0 = 0; k0 < limit; k0 += 64) {
      const int key = k0 + lane;
      float s = -INFINITY;
      int64_t vbase = -1;
      if (key < limit) {
        const int64_t blk = btrow[key / p.BS];
        if (blk >= 0 && blk < p.num_blocks) {
          const int64_t slot = key % p.BS;
          vbase = blk * p.v_sb + slot * p.v_ss + (int64_t)kvh * p.v_sh;
          const float* kp = kc + blk * p.k_sb + slot * p.k_ss + (int64_t)kvh * p.k_sh;
          float dot = 0.f;
          for (int d = 0; d < D; d += 4) {
            const float4 kv4 = *(const float4*)(kp + d);
            dot = __builtin_fmaf(s_q[d], kv4.x, dot);
            dot = __builtin_fmaf(s_q[d + 1], kv4.y, dot);
            dot = __builtin_fmaf(s_q[d + 2], kv4.z, dot);
            dot = __builtin_fmaf(s_q[d + 3], kv4.w, dot);
          }
          s = dot * p.qk_scale;
        }
      }
      float mx = s;
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
      const float m_new = fmaxf(m, mx);
      const float m_safe = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = exp2f(m - m_safe);
      const float pk = exp2f(s - m_safe);
      float ps = pk;
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) ps += __shfl_xor(ps, o);
      l = l * alpha + ps;
      m = m_new;
#pragma unroll
      for (int x = 0; x < DPL; ++x) acc[x] *= alpha;
      const int nk = min(64, limit - k0);
      for (int kk = 0; kk < nk; ++kk) {
        const float pw = __shfl(pk, kk);
        const int64_t vb = __shfl(vbase, kk);
        if (vb < 0) continue;  // empty page: weight is 0 and there is nothing to read
        const float* vp = vc + vb;
#pragma unroll
        for (int x = 0; x < DPL; ++x) {
          const int d = lane + 64 * x;
          if (d < D) acc[x] = __builtin_fmaf(pw, vp[d], acc[x]);
        }
      }
    }
    const float inv = 1.f / (l == 0.f ? 1.f : l);
    float* orow = (float*)p.out + tok * p.o_ts + (int64_t)head * p.o_hs;
#pragma unroll
    for (int x = 0; x < DPL; ++x) {
      const int d = lane + 64 * x;
      if (d < D) orow[d] = acc[x] * inv;
    }
  }
}

int launch_paged_attention_f32(const PAParams& p, int32_t D, int32_t max_q, hipStream_t s, LaunchLog& log) {
  dim3 grid(p.B, p.H, (max_q + kRowsPerWG - 1) / kRowsPerWG);
  if (D <= 64)
    hipLaunchKernelGGL((pa_f32_kernel<1>), grid, dim3(64), 0, s, p, D);
  else if (D <= 128)
    hipLaunchKernelGGL((pa_f32_kernel<2>), grid, dim3(64), 0, s, p, D);
  else
    hipLaunchKernelGGL((pa_f32_kernel<4>), grid, dim3(64), 0, s, p, D);
  const int err = (int)hipGetLastError();
  if (!err) log.after_launch(4, s);
  return err;
}

}  // namespace kvh

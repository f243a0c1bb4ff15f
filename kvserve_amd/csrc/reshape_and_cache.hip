// reshape_and_cache: scatter this step's K/V rows into the paged pool, bit for bit.
// Semantics: TorchAttention.write_kv, src/kvserve/attention.py:39-45
//   k_cache.view(-1, Hkv, D)[slots] = k ; v_cache.view(-1, Hkv, D)[slots] = v
// with slot s -> (block s / BS, offset s % BS) (src/kvserve/kv_cache.py:155-157).
//
// HBM-bound copy: every byte of k and v is read once and written once. A workgroup copies the
// K and V rows of `tpw` consecutive tokens (2 Hkv D e bytes each, 4 KB at the Llama-8B shape),
// 16-byte vectors per thread, rows contiguous per (slot, head) so every access is coalesced.
// A thread issues the loads of its vector of every token of the workgroup (and the tokens'
// slots, which the source addresses do not depend on) before the first store; tokens per
// workgroup grow with the batch (1 for a decode step, 4 for a 2048-token mixed step) so large
// steps launch fewer, fuller workgroups. v may be a strided
// view of the fused QKV output (token stride (H + 2 Hkv) D); only its rows are touched.
// Slots outside the pool are skipped (the reference's index_put_ would raise or wrap).
#include <type_traits>

#include "kvh_device.h"
#include "kvh_internal.h"

namespace kvh {

// Byte offset of a slot's (block, offset) in a cache with byte strides sb, ss; 32-bit division
// when every slot fits (a uniform branch on the pool size).
__device__ __forceinline__ int64_t slot_offset(int64_t slot, int64_t num_slots, int BS, int64_t sb, int64_t ss) {
  if (num_slots <= 0x7fffffffLL) {
    const uint32_t s32 = (uint32_t)slot, b = s32 / (uint32_t)BS;
    return (int64_t)b * sb + (int64_t)(s32 - b * (uint32_t)BS) * ss;
  }
  return (slot / BS) * sb + (slot % BS) * ss;
}

// Tokens per workgroup for a batch of T tokens: about 512 workgroups or more, at most 4
// tokens each (the loads a thread keeps in flight).
constexpr int kRacMaxTokens = 4;
inline int rac_tokens_per_wg(int64_t T) { return T >= 4 * 512 ? 4 : (T >= 2 * 512 ? 2 : 1); }

// Thread `tid` of a workgroup copies vector r = tid + 256 c (c = 0, 1, ...) of each of the
// workgroup's tokens' K|V rows (per_tok vectors: K heads, then V heads); its (tensor, head,
// offset) is computed once per c, the tokens' slots and sources are loaded together, and the
// stores follow.
template <int VB>  // bytes per thread: 16 (vector path) or the element size
__global__ __launch_bounds__(256) void reshape_and_cache_kernel(
    const uint8_t* k, int64_t k_ts, int64_t k_hs, const uint8_t* v, int64_t v_ts, int64_t v_hs,
    uint8_t* kc, int64_t k_sb, int64_t k_ss, int64_t k_sh, uint8_t* vc, int64_t v_sb, int64_t v_ss,
    int64_t v_sh, const int64_t* slots, int64_t num_slots, int Hkv, int row_bytes, int BS, int eb, int64_t T,
    int tpw) {
  typedef std::conditional_t<VB == 16, u32x4, std::conditional_t<VB == 4, uint32_t, uint16_t>> vec_t;
  // strides arrive in elements; addresses are formed in bytes
  const int vpr = row_bytes / VB;  // vectors per (token, head) row
  const int per_tensor = Hkv * vpr;
  const int per_tok = 2 * per_tensor;
  const int64_t t0 = (int64_t)blockIdx.x * tpw;
  const int nt = (int)min((int64_t)tpw, T - t0);
  int64_t slot[kRacMaxTokens];
#pragma unroll
  for (int j = 0; j < kRacMaxTokens; ++j) slot[j] = j < nt ? slots[t0 + j] : -1;
  for (int r0 = threadIdx.x; r0 < per_tok; r0 += 256) {
    const bool is_v = r0 >= per_tensor;
    const int r = is_v ? r0 - per_tensor : r0;
    const int h = r / vpr, x = r % vpr;
    const uint8_t* src = (is_v ? v + (t0 * v_ts + (int64_t)h * v_hs) * eb : k + (t0 * k_ts + (int64_t)h * k_hs) * eb) +
                         x * VB;
    const int64_t src_ts = (is_v ? v_ts : k_ts) * eb;
    uint8_t* const cbase = (is_v ? vc + (int64_t)h * v_sh * eb : kc + (int64_t)h * k_sh * eb) + x * VB;
    const int64_t sb = (is_v ? v_sb : k_sb) * eb, ss = (is_v ? v_ss : k_ss) * eb;
    vec_t val[kRacMaxTokens];
#pragma unroll
    for (int j = 0; j < kRacMaxTokens; ++j)
      if (j < nt) val[j] = *(const vec_t*)(src + j * src_ts);
#pragma unroll
    for (int j = 0; j < kRacMaxTokens; ++j) {
      if (j >= nt || slot[j] < 0 || slot[j] >= num_slots) continue;
      *(vec_t*)(cbase + slot_offset(slot[j], num_slots, BS, sb, ss)) = val[j];
    }
  }
}

// FP8 cache (kvh_reshape_and_cache_fp8): the same scatter, each element stored as
// e4m3(clamp(x / scale, -448, 448)) (fp8_prep / fp8_pack4). A thread converts 8 consecutive
// elements of one (token, head) row: one 16-byte load (two for fp32 sources), one 8-byte store;
// workgroups take tpw tokens, a thread's granules of all of them loaded before any store, as in
// the 16-bit copy.
template <int DT>  // source type: 0 fp32, 1 fp16, 2 bf16
__global__ __launch_bounds__(256) void reshape_and_cache_fp8_kernel(
    const uint8_t* k, int64_t k_ts, int64_t k_hs, const uint8_t* v, int64_t v_ts, int64_t v_hs, uint8_t* kc,
    int64_t k_sb, int64_t k_ss, int64_t k_sh, uint8_t* vc, int64_t v_sb, int64_t v_ss, int64_t v_sh,
    const int64_t* slots, int64_t num_slots, int Hkv, int D, int BS, float k_scale, float v_scale, int64_t T,
    int tpw) {
  constexpr int EB = DT == 0 ? 4 : 2;
  const int vpr = D / 8;
  const int per_tensor = Hkv * vpr;
  const int per_tok = 2 * per_tensor;
  const int64_t t0 = (int64_t)blockIdx.x * tpw;
  const int nt = (int)min((int64_t)tpw, T - t0);
  int64_t slot[kRacMaxTokens];
#pragma unroll
  for (int j = 0; j < kRacMaxTokens; ++j) slot[j] = j < nt ? slots[t0 + j] : -1;
  for (int r0 = threadIdx.x; r0 < per_tok; r0 += 256) {
    const bool is_v = r0 >= per_tensor;
    const int r = is_v ? r0 - per_tensor : r0;
    const int h = r / vpr, x = (r % vpr) * 8;
    const uint8_t* src = is_v ? v + (t0 * v_ts + (int64_t)h * v_hs + x) * EB : k + (t0 * k_ts + (int64_t)h * k_hs + x) * EB;
    const int64_t src_ts = (is_v ? v_ts : k_ts) * EB;
    uint8_t* const cbase = is_v ? vc + (int64_t)h * v_sh + x : kc + (int64_t)h * k_sh + x;
    const int64_t sb = is_v ? v_sb : k_sb, ss = is_v ? v_ss : k_ss;
    const float scale = is_v ? v_scale : k_scale;
    float f[kRacMaxTokens][8];
#pragma unroll
    for (int j = 0; j < kRacMaxTokens; ++j) {
      if (j >= nt) continue;
      const uint8_t* sj = src + j * src_ts;
      if constexpr (DT == 0) {
        const f32x4 a = *(const f32x4*)sj, b = *(const f32x4*)(sj + 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          f[j][i] = a[i];
          f[j][4 + i] = b[i];
        }
      } else {
        const u32x4 w = *(const u32x4*)sj;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const uint16_t e = (uint16_t)(w[i / 2] >> (16 * (i & 1)));
          f[j][i] = DT == 2 ? BF16::to_f32(e) : F16::to_f32(e);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < kRacMaxTokens; ++j) {
      if (j >= nt || slot[j] < 0 || slot[j] >= num_slots) continue;
      float g[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) g[i] = fp8_prep(f[j][i], scale);
      *(u32x2*)(cbase + slot_offset(slot[j], num_slots, BS, sb, ss)) =
          u32x2{fp8_pack4(g[0], g[1], g[2], g[3]), fp8_pack4(g[4], g[5], g[6], g[7])};
    }
  }
}

int launch_reshape_and_cache_fp8(const void* k, int64_t k_ts, int64_t k_hs, const void* v, int64_t v_ts,
                                 int64_t v_hs, void* kc, const int64_t* kcs, void* vc, const int64_t* vcs,
                                 const int64_t* slots, int64_t T, int64_t num_blocks, int32_t Hkv, int32_t D,
                                 int32_t BS, int32_t dtype, float k_scale, float v_scale, hipStream_t s) {
  if (T == 0) return 0;
  const int tpw = rac_tokens_per_wg(T);
  dim3 grid((unsigned)((T + tpw - 1) / tpw));
  const int64_t num_slots = num_blocks * BS;
#define KVH_LAUNCH_RAC8(DT)                                                                                        \
  hipLaunchKernelGGL((reshape_and_cache_fp8_kernel<DT>), grid, dim3(256), 0, s, (const uint8_t*)k, k_ts, k_hs,    \
                     (const uint8_t*)v, v_ts, v_hs, (uint8_t*)kc, kcs[0], kcs[1], kcs[2], (uint8_t*)vc, vcs[0],     \
                     vcs[1], vcs[2], slots, num_slots, Hkv, D, BS, k_scale, v_scale, T, tpw)
  if (dtype == 2)
    KVH_LAUNCH_RAC8(2);
  else if (dtype == 1)
    KVH_LAUNCH_RAC8(1);
  else
    KVH_LAUNCH_RAC8(0);
#undef KVH_LAUNCH_RAC8
  return (int)hipGetLastError();
}

int launch_reshape_and_cache(const void* k, int64_t k_ts, int64_t k_hs, const void* v, int64_t v_ts,
                             int64_t v_hs, void* kc, const int64_t* kcs, void* vc, const int64_t* vcs,
                             const int64_t* slots, int64_t T, int64_t num_blocks, int32_t Hkv, int32_t D,
                             int32_t BS, int32_t elem_bytes, bool vec16, hipStream_t s) {
  if (T == 0) return 0;
  const int row_bytes = D * elem_bytes;
  const int vb = vec16 ? 16 : elem_bytes;
  const int tpw = rac_tokens_per_wg(T);
  dim3 grid((unsigned)((T + tpw - 1) / tpw));
  const int64_t num_slots = num_blocks * BS;
#define KVH_LAUNCH_RAC(VB)                                                                                     \
  hipLaunchKernelGGL((reshape_and_cache_kernel<VB>), grid, dim3(256), 0, s, (const uint8_t*)k, k_ts, k_hs,    \
                     (const uint8_t*)v, v_ts, v_hs, (uint8_t*)kc, kcs[0], kcs[1], kcs[2], (uint8_t*)vc, vcs[0], \
                     vcs[1], vcs[2], slots, num_slots, Hkv, row_bytes, BS, elem_bytes, T, tpw)
  if (vb == 16)
    KVH_LAUNCH_RAC(16);
  else if (vb == 4)
    KVH_LAUNCH_RAC(4);
  else
    KVH_LAUNCH_RAC(2);
#undef KVH_LAUNCH_RAC
  return (int)hipGetLastError();
}

}  // namespace kvh

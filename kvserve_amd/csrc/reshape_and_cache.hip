// reshape_and_cache: scatter this step's K/V rows into the paged pool, bit for bit.
// Semantics: TorchAttention.write_kv, src/kvserve/attention.py:39-45
//   k_cache.view(-1, Hkv, D)[slots] = k ; v_cache.view(-1, Hkv, D)[slots] = v
// with slot s -> (block s / BS, offset s % BS) (src/kvserve/kv_cache.py:155-157).
//
// HBM-bound copy: every byte of k and v is read once and written once. Grid (T, chunks):
// one workgroup per token (its K and V rows are 2 * Hkv * D * e bytes, 4 KB at the Llama-8B
// shape = one 256-thread workgroup of 16-byte vectors), so a token's whole write is
// contiguous per (slot, head) row and fully coalesced. v may be a strided view of the
// fused QKV output (token stride (H + 2 Hkv) D); only its rows are touched.
// Slots outside the pool are skipped (the reference's index_put_ would raise or wrap).
#include "kvh_device.h"
#include "kvh_internal.h"

namespace kvh {

template <int VB>  // bytes per thread: 16 (vector path) or the element size
__global__ __launch_bounds__(256) void reshape_and_cache_kernel(
    const uint8_t* k, int64_t k_ts, int64_t k_hs, const uint8_t* v, int64_t v_ts, int64_t v_hs,
    uint8_t* kc, int64_t k_sb, int64_t k_ss, int64_t k_sh, uint8_t* vc, int64_t v_sb, int64_t v_ss,
    int64_t v_sh, const int64_t* slots, int64_t num_slots, int Hkv, int row_bytes, int BS, int eb) {
  // strides arrive in elements; addresses are formed in bytes
  const int64_t t = blockIdx.x;
  const int vpr = row_bytes / VB;  // vectors per (token, head) row
  const int per_tensor = Hkv * vpr;
  const int idx = blockIdx.y * 256 + threadIdx.x;
  if (idx >= 2 * per_tensor) return;
  const int64_t slot = slots[t];
  if (slot < 0 || slot >= num_slots) return;
  const int64_t blk = slot / BS, off = slot % BS;
  const bool is_v = idx >= per_tensor;
  const int r = is_v ? idx - per_tensor : idx;
  const int h = r / vpr, x = r % vpr;
  const uint8_t* src;
  uint8_t* dst;
  if (is_v) {
    src = v + (t * v_ts + (int64_t)h * v_hs) * eb + x * VB;
    dst = vc + (blk * v_sb + off * v_ss + (int64_t)h * v_sh) * eb + x * VB;
  } else {
    src = k + (t * k_ts + (int64_t)h * k_hs) * eb + x * VB;
    dst = kc + (blk * k_sb + off * k_ss + (int64_t)h * k_sh) * eb + x * VB;
  }
  if constexpr (VB == 16) {
    *(u32x4*)dst = *(const u32x4*)src;
  } else if constexpr (VB == 4) {
    *(uint32_t*)dst = *(const uint32_t*)src;
  } else {
    *(uint16_t*)dst = *(const uint16_t*)src;
  }
}

// FP8 cache (kvh_reshape_and_cache_fp8): the same scatter, each element stored as
// e4m3(clamp(x / scale, -448, 448)) (fp8_prep / fp8_pack4). A thread converts 8 consecutive
// elements of one (token, head) row: one 16-byte load (two for fp32 sources), one 8-byte store.
template <int DT>  // source type: 0 fp32, 1 fp16, 2 bf16
__global__ __launch_bounds__(256) void reshape_and_cache_fp8_kernel(
    const uint8_t* k, int64_t k_ts, int64_t k_hs, const uint8_t* v, int64_t v_ts, int64_t v_hs, uint8_t* kc,
    int64_t k_sb, int64_t k_ss, int64_t k_sh, uint8_t* vc, int64_t v_sb, int64_t v_ss, int64_t v_sh,
    const int64_t* slots, int64_t num_slots, int Hkv, int D, int BS, float k_scale, float v_scale) {
  constexpr int EB = DT == 0 ? 4 : 2;
  const int64_t t = blockIdx.x;
  const int vpr = D / 8;
  const int per_tensor = Hkv * vpr;
  const int idx = blockIdx.y * 256 + threadIdx.x;
  if (idx >= 2 * per_tensor) return;
  const int64_t slot = slots[t];
  if (slot < 0 || slot >= num_slots) return;
  const int64_t blk = slot / BS, off = slot % BS;
  const bool is_v = idx >= per_tensor;
  const int r = is_v ? idx - per_tensor : idx;
  const int h = r / vpr, x = (r % vpr) * 8;
  const uint8_t* src = is_v ? v + (t * v_ts + (int64_t)h * v_hs + x) * EB : k + (t * k_ts + (int64_t)h * k_hs + x) * EB;
  uint8_t* dst = is_v ? vc + blk * v_sb + off * v_ss + (int64_t)h * v_sh + x : kc + blk * k_sb + off * k_ss + (int64_t)h * k_sh + x;
  const float scale = is_v ? v_scale : k_scale;
  float f[8];
  if constexpr (DT == 0) {
    const f32x4 a = *(const f32x4*)src, b = *(const f32x4*)(src + 16);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[i] = a[i];
      f[4 + i] = b[i];
    }
  } else {
    const u32x4 w = *(const u32x4*)src;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint16_t e = (uint16_t)(w[i / 2] >> (16 * (i & 1)));
      f[i] = DT == 2 ? BF16::to_f32(e) : F16::to_f32(e);
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) f[i] = fp8_prep(f[i], scale);
  *(u32x2*)dst = u32x2{fp8_pack4(f[0], f[1], f[2], f[3]), fp8_pack4(f[4], f[5], f[6], f[7])};
}

int launch_reshape_and_cache_fp8(const void* k, int64_t k_ts, int64_t k_hs, const void* v, int64_t v_ts,
                                 int64_t v_hs, void* kc, const int64_t* kcs, void* vc, const int64_t* vcs,
                                 const int64_t* slots, int64_t T, int64_t num_blocks, int32_t Hkv, int32_t D,
                                 int32_t BS, int32_t dtype, float k_scale, float v_scale, hipStream_t s) {
  if (T == 0) return 0;
  const int total = 2 * Hkv * (D / 8);
  dim3 grid((unsigned)T, (unsigned)((total + 255) / 256));
  const int64_t num_slots = num_blocks * BS;
#define KVH_LAUNCH_RAC8(DT)                                                                                        \
  hipLaunchKernelGGL((reshape_and_cache_fp8_kernel<DT>), grid, dim3(256), 0, s, (const uint8_t*)k, k_ts, k_hs,    \
                     (const uint8_t*)v, v_ts, v_hs, (uint8_t*)kc, kcs[0], kcs[1], kcs[2], (uint8_t*)vc, vcs[0],     \
                     vcs[1], vcs[2], slots, num_slots, Hkv, D, BS, k_scale, v_scale)
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
  const int total = 2 * Hkv * (row_bytes / vb);
  dim3 grid((unsigned)T, (unsigned)((total + 255) / 256));
  const int64_t num_slots = num_blocks * BS;
#define KVH_LAUNCH_RAC(VB)                                                                                     \
  hipLaunchKernelGGL((reshape_and_cache_kernel<VB>), grid, dim3(256), 0, s, (const uint8_t*)k, k_ts, k_hs,    \
                     (const uint8_t*)v, v_ts, v_hs, (uint8_t*)kc, kcs[0], kcs[1], kcs[2], (uint8_t*)vc, vcs[0], \
                     vcs[1], vcs[2], slots, num_slots, Hkv, row_bytes, BS, elem_bytes)
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

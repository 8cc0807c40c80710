// Decode-step rotary embedding fused with the paged KV append.
//
// The reference applies RoPE to the projected q and k (models/modeling_llama.py:
// 460-465, HF apply_rotary_pos_emb) and then appends k and v to the paged cache
// (write_blocks_vectorized, page_table.py:167-209).  Here one kernel reads the
// fused q|k|v projection row of every candidate once, writes rotated q for the
// attention kernel and scatters rotated k and v into their page slot.
//
// Numerics follow the eager tensor code exactly for 16-bit storage:
//   out = round(round(x * cos) + round(rotate_half(x) * sin)),
// rotate_half(x)[i] = -x[i + D/2] for i < D/2, x[i - D/2] otherwise.

#include "common.h"

namespace be {

template <typename T>
__device__ __forceinline__ float rnd(float x) { return to_f32(from_f32<T>(x)); }

// Four consecutive 16-bit elements as one 8-byte access (the host checks the
// alignment of every row these address).
typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
template <typename T>
__device__ __forceinline__ void load4(const T* p, T (&v)[4]) {
  const u16x4 u = *reinterpret_cast<const u16x4*>(p);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint16_t b = u[e];
    v[e] = __builtin_bit_cast(T, b);
  }
}
template <typename T>
__device__ __forceinline__ void store4(T* p, const T (&v)[4]) {
  u16x4 u;
#pragma unroll
  for (int e = 0; e < 4; ++e) u[e] = __builtin_bit_cast(uint16_t, v[e]);
  *reinterpret_cast<u16x4*>(p) = u;
}

// One thread per (candidate, head, 4 rotation pairs).  Heads [0, hq) are q,
// [hq, hq + hkv) are k, [hq + hkv, hq + 2 hkv) are v (copied, not rotated).
template <typename T>
__global__ __launch_bounds__(256) void rope_append_kernel(const T* qkv, int64_t qkv_sn, int n, int hq, int hkv,
                                                         int d, const int64_t* positions, const T* cos_t,
                                                         const T* sin_t, int max_pos, T* q_out, T* kv,
                                                         int num_pages, int page_size, const int32_t* page_idx,
                                                         const int32_t* slot, int32_t* err) {
  const int half = d / 2, quads = half / 4;
  const int heads = hq + 2 * hkv;
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t total = (int64_t)n * heads * quads;
  if (gid >= total) return;
  const int qd = (int)(gid % quads);
  const int h = (int)((gid / quads) % heads);
  const int i = (int)(gid / ((int64_t)quads * heads));
  const T* src = qkv + (int64_t)i * qkv_sn + (int64_t)h * d;
  const int j0 = qd * 4;
  T lo[4], hi[4];
  load4(src + j0, lo);
  load4(src + half + j0, hi);
  if (h < hq + hkv) {
    const int64_t p = positions[i];
    if (p < 0 || p >= max_pos) {
      if (err && qd == 0 && h == 0) atomicAdd(err, 1);
      return;
    }
    T cl[4], ch[4], sl[4], sh[4];
    load4(cos_t + p * d + j0, cl);
    load4(cos_t + p * d + half + j0, ch);
    load4(sin_t + p * d + j0, sl);
    load4(sin_t + p * d + half + j0, sh);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float xl = to_f32(lo[e]), xh = to_f32(hi[e]);
      const float ol = rnd<T>(rnd<T>(xl * to_f32(cl[e])) + rnd<T>(-xh * to_f32(sl[e])));
      const float oh = rnd<T>(rnd<T>(xh * to_f32(ch[e])) + rnd<T>(xl * to_f32(sh[e])));
      lo[e] = from_f32<T>(ol);
      hi[e] = from_f32<T>(oh);
    }
  }
  T* dst;
  if (h < hq) {
    dst = q_out + ((int64_t)i * hq + h) * d;
  } else {
    const int pg = page_idx[i], sl = slot[i];
    if (pg < 0 || pg >= num_pages || sl < 0 || sl >= page_size) {
      if (err && qd == 0 && h == hq) atomicAdd(err, 1);
      return;
    }
    const int kvsel = (h < hq + hkv) ? 0 : 1;
    const int kh = (h < hq + hkv) ? h - hq : h - hq - hkv;
    dst = kv + ((((int64_t)pg * 2 + kvsel) * page_size + sl) * hkv + kh) * d;
  }
  store4(dst + j0, lo);
  store4(dst + half + j0, hi);
}

}  // namespace be

extern "C" int be_rope_qkv_append(const void* qkv, int64_t qkv_stride_n, int dtype, int n, int num_qo_heads,
                                  int num_kv_heads, int head_dim, const int64_t* positions, const void* cos_table,
                                  const void* sin_table, int max_position, void* q_out, void* kv_layer, int num_pages,
                                  int page_size, const int32_t* page_idx, const int32_t* slot, int32_t* err_count,
                                  void* stream) {
  BE_REQUIRE(n >= 0, "n must be >= 0");
  if (n == 0) return BE_OK;
  BE_REQUIRE(qkv && positions && cos_table && sin_table && q_out && kv_layer && page_idx && slot, "null pointer");
  BE_REQUIRE(dtype == BE_F16 || dtype == BE_BF16, "rope append supports fp16 / bf16 storage");
  BE_REQUIRE(num_qo_heads > 0 && num_kv_heads > 0 && head_dim > 0 && head_dim % 8 == 0, "bad head shape");
  BE_REQUIRE(qkv_stride_n >= (int64_t)(num_qo_heads + 2 * num_kv_heads) * head_dim, "qkv row stride too small");
  BE_REQUIRE(qkv_stride_n % 4 == 0 && (reinterpret_cast<uintptr_t>(qkv) & 7) == 0 &&
                 (reinterpret_cast<uintptr_t>(cos_table) & 7) == 0 && (reinterpret_cast<uintptr_t>(sin_table) & 7) == 0 &&
                 (reinterpret_cast<uintptr_t>(q_out) & 7) == 0 && (reinterpret_cast<uintptr_t>(kv_layer) & 7) == 0,
             "qkv, tables, q_out and the cache must be 8-byte aligned with a qkv row stride that is a multiple of 4");
  BE_REQUIRE(num_pages > 0 && page_size > 0 && max_position > 0, "bad cache / table shape");
  const int64_t total = (int64_t)n * (num_qo_heads + 2 * num_kv_heads) * (head_dim / 8);
  const unsigned blocks = (unsigned)((total + 255) / 256);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (dtype == BE_BF16)
    be::rope_append_kernel<be::bf16_t><<<blocks, 256, 0, st>>>(
        (const be::bf16_t*)qkv, qkv_stride_n, n, num_qo_heads, num_kv_heads, head_dim, positions,
        (const be::bf16_t*)cos_table, (const be::bf16_t*)sin_table, max_position, (be::bf16_t*)q_out,
        (be::bf16_t*)kv_layer, num_pages, page_size, page_idx, slot, err_count);
  else
    be::rope_append_kernel<be::f16_t><<<blocks, 256, 0, st>>>(
        (const be::f16_t*)qkv, qkv_stride_n, n, num_qo_heads, num_kv_heads, head_dim, positions,
        (const be::f16_t*)cos_table, (const be::f16_t*)sin_table, max_position, (be::f16_t*)q_out,
        (be::f16_t*)kv_layer, num_pages, page_size, page_idx, slot, err_count);
  BE_HIP_CHECK(hipGetLastError());
  return BE_OK;
}

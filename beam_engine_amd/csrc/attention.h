// Declarations shared by the decode attention sources (gfx950): the planner's
// group list, MFMA operand helpers, and the persistent streaming kernel's plan
// and run entry points (attn_stream.hip).
#pragma once

#include <vector>

#include "common.h"

namespace be {

constexpr int kPlanHeader = 16;    // int32 words of live counts at the start of a plan
constexpr int kHdrItems = 0, kHdrMerge = 1, kHdrZero = 2, kHdrRows = 3, kHdrTailItems = 4;

// One paged group of one cascade level after validation: queries [q0, q1)
// attend kv_len tokens whose pages start at page_base of the plan's
// concatenated page list.
struct Group {
  int level, q0, q1, page_base, kv_len;
};

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

typedef short v8s __attribute__((ext_vector_type(8)));
typedef short v4s __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

// Reductions over the four lanes l, l ^ 16, l ^ 32, l ^ 48 (the four 16-lane
// rows of a wave that hold one MFMA column), on the VALU: v_permlane16_swap
// exchanges odd and even 16-lane rows of its two operands and
// v_permlane32_swap the wave's halves, so with both operands equal to x, one
// result is x and the other the partner lane's x in every lane.  (A
// __shfl_xor is an LDS permute whose wait also waits for the wave's
// outstanding LDS reads.)  Vector elements are copied out before the bit
// casts: a bit cast of an element expression reads element 0.
__device__ __forceinline__ float rows4_max(float x) {
  typedef unsigned int u2 __attribute__((ext_vector_type(2)));
  const unsigned xb = __float_as_uint(x);
  const u2 a = __builtin_amdgcn_permlane16_swap(xb, xb, false, false);
  const unsigned a0 = a.x, a1 = a.y;
  const unsigned yb = __float_as_uint(fmaxf(__uint_as_float(a0), __uint_as_float(a1)));
  const u2 b = __builtin_amdgcn_permlane32_swap(yb, yb, false, false);
  const unsigned b0 = b.x, b1 = b.y;
  return fmaxf(__uint_as_float(b0), __uint_as_float(b1));
}
// The same lanes' sum; every lane gets the bit-identical (x0 + x1) + (x2 + x3).
__device__ __forceinline__ float rows4_sum(float x) {
  typedef unsigned int u2 __attribute__((ext_vector_type(2)));
  const unsigned xb = __float_as_uint(x);
  const u2 a = __builtin_amdgcn_permlane16_swap(xb, xb, false, false);
  const unsigned a0 = a.x, a1 = a.y;
  const unsigned yb = __float_as_uint(__uint_as_float(a0) + __uint_as_float(a1));
  const u2 b = __builtin_amdgcn_permlane32_swap(yb, yb, false, false);
  const unsigned b0 = b.x, b1 = b.y;
  return __uint_as_float(b0) + __uint_as_float(b1);
}

// S^T tile: v_mfma_f32_16x16x32 on 16-bit operands.
template <typename T> __device__ __forceinline__ v4f mfma_qk(v8s a, v8s b, v4f c);
template <> __device__ __forceinline__ v4f mfma_qk<bf16_t>(v8s a, v8s b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
template <> __device__ __forceinline__ v4f mfma_qk<f16_t>(v8s a, v8s b, v4f c) {
  typedef _Float16 v8h __attribute__((ext_vector_type(8)));
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, a), __builtin_bit_cast(v8h, b), c, 0, 0, 0);
}
// O^T += V^T P^T: v_mfma_f32_16x16x16 on 16-bit operands.
template <typename T> __device__ __forceinline__ v4f mfma_pv(v4s a, v4s b, v4f c);
template <> __device__ __forceinline__ v4f mfma_pv<bf16_t>(v4s a, v4s b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}
template <> __device__ __forceinline__ v4f mfma_pv<f16_t>(v4s a, v4s b, v4f c) {
  typedef _Float16 v4h __attribute__((ext_vector_type(4)));
  return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(v4h, a), __builtin_bit_cast(v4h, b), c, 0, 0, 0);
}

template <typename T> __device__ __forceinline__ uint16_t pack16(float x);
template <> __device__ __forceinline__ uint16_t pack16<bf16_t>(float x) { return f32_to_bf16_bits(x); }
template <> __device__ __forceinline__ uint16_t pack16<f16_t>(float x) {
  return __builtin_bit_cast(uint16_t, (_Float16)x);
}

// ---------------------------------------------------------------- streaming kernel
// True when the streaming kernel serves this shape (16-bit storage, head_dim
// 128, GQA group <= 64, page size a multiple of 16).
bool stream_eligible(int dtype, int head_dim, int group, int page_size, int flags);

// Writes the streaming plan for `groups` (validated by attn_plan, pages
// concatenated level by level into total_pages entries) into out[0..cap) and
// fills the layout fields of info.  Returns BE_ERR_UNSUPPORTED (without
// setting an error) when a workgroup would need more segments than its LDS
// table holds; the caller then plans for the tile kernel instead.
int stream_plan(const std::vector<Group>& groups, const be_level* levels, int num_levels, int64_t total_pages,
                int num_queries, int hq, int hkv, int d, int page_size, int num_pages, int dtype, int num_cus,
                int flags, const be_plan_caps* caps, int32_t* out, int64_t cap, be_attn_plan_info* info);

// Launches the streaming attention kernel (phases & BE_RUN_ATTENTION) and the
// tail-and-merge kernel (phases & BE_RUN_MERGE) of a kernel == 2 plan.
int stream_run(const be_attn_plan_info* info, const int32_t* plan, void* partials, const void* q, int64_t q_sn,
               int64_t q_sh, const void* kv, void* out, int64_t o_sn, int64_t o_sh, float* lse, float sm_scale,
               int phases, hipStream_t st);

// ---------------------------------------------------------------- row-block kernel
// Writes the merge-free row-block plan (attn_rows.hip) for `groups` into
// out[0..cap) and fills its layout fields of info (kernel 3).
int rows_plan(const std::vector<Group>& groups, const be_level* levels, int num_levels, int64_t total_pages,
              int num_queries, int hq, int hkv, int page_size, int num_cus, int32_t* out, int64_t cap,
              be_attn_plan_info* info);

// True when the row-block plan is expected to beat the streaming plan: every
// block's passes re-read the groups it shares with other blocks (from L2),
// so it pays where the streaming plan's fixed costs (partials, a second
// kernel) dominate.
bool rows_preferred(const std::vector<Group>& groups, int num_queries, int g, int num_cus);

// Launches the row-block kernel of a kernel == 3 plan (phases & BE_RUN_ATTENTION;
// it has no merge phase).
int rows_run(const be_attn_plan_info* info, const int32_t* plan, const void* q, int64_t q_sn, int64_t q_sh,
             const void* kv, void* out, int64_t o_sn, int64_t o_sh, float* lse, float sm_scale, int phases,
             hipStream_t st);

}  // namespace be

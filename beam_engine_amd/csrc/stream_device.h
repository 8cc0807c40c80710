// Device helpers shared by the streaming decode-attention kernels (gfx950):
// direct global->LDS loads, explicit vmcnt waits, 16-bit packing, segment
// records in registers, and the per-wave MFMA tile step of a 64-token tile
// (K / V rows of 256 bytes in LDS, 16-byte chunks XOR-swizzled by row).
#pragma once

#include "attention.h"

namespace be {
namespace stream {

constexpr int kD = 128;                       // head_dim served
constexpr int kTok = 64;                      // tokens per tile

typedef __attribute__((address_space(3))) void* lds_ptr_t;
typedef __attribute__((address_space(3))) v4s* lds_v4s_t;

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(lds_ptr_t)p;
}

// Direct global->LDS loads: lane l's bytes land at LDS byte address m0 + size * l
// (lds must be wave-uniform).  They are issued from inline asm so that the
// compiler's wait insertion does not treat every later LDS read as dependent
// on them (it would wait for all outstanding loads); completion is tracked by
// the explicit vmcnt waits.  Wait states: an M0 write needs one before an
// LDS-DMA instruction reads it; an SGPR written by a VALU instruction
// (readfirstlane) needs five before a vector memory instruction reads it.
__device__ __forceinline__ void dma16(const void* src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(src), "s"(lds)
               : "memory", "m0");
}
// SGPR base (wave-uniform) + 32-bit unsigned VGPR byte offset
__device__ __forceinline__ void dma16_sv(uint64_t base, uint32_t voff, uint32_t lds) {
  // readfirstlane returns int: zero-extend each half through uint32_t
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(base >> 32));
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)base);
  const uint64_t sbase = ((uint64_t)hi << 32) | (uint64_t)lo;
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 4\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(voff), "s"(sbase), "s"(lds)
               : "memory", "m0");
}
__device__ __forceinline__ void dma4(const void* src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off"
               :
               : "v"(src), "s"(lds)
               : "memory", "m0");
}

// s_waitcnt vmcnt(n) (gfx9 encoding: vmcnt[3:0] | expcnt 7 | lgkmcnt 15 | vmcnt[5:4] << 14).
// n is the number of newer vector memory operations that may stay
// outstanding; vmcnt retires operations in issue order.  Dispatched by a
// binary tree of scalar branches (n is wave-uniform).
#define BE_VMCNT(n) (((n) & 15) | (7 << 4) | (15 << 8) | (((n) >> 4) << 14))
template <int LO, int HI>
__device__ __forceinline__ void wait_tree(int n) {
  if constexpr (LO == HI) {
    __builtin_amdgcn_s_waitcnt(BE_VMCNT(LO));
  } else {
    constexpr int MID = (LO + HI) / 2;
    if (n <= MID) wait_tree<LO, MID>(n);
    else wait_tree<MID + 1, HI>(n);
  }
}
__device__ __forceinline__ void wait_vmcnt(int n) { wait_tree<0, 31>(n < 31 ? n : 31); }

// Bare workgroup barrier (after explicit vmcnt waits for direct loads).
__device__ __forceinline__ void lds_fence() {
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Workgroup barrier after this wave's LDS writes have completed (s_waitcnt
// lgkmcnt(0), then s_barrier; vector memory loads stay in flight).
__device__ __forceinline__ void lds_sync() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

__device__ __forceinline__ int rfl(int x) { return __builtin_amdgcn_readfirstlane(x); }

// Two floats -> two 16-bit values (round to nearest even) in one word.
template <typename T> __device__ __forceinline__ uint32_t pack2(float a, float b);
template <> __device__ __forceinline__ uint32_t pack2<bf16_t>(float a, float b) {
  typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
  typedef float f2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2){a, b}, bf2));
}
template <> __device__ __forceinline__ uint32_t pack2<f16_t>(float a, float b) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  typedef float f2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2){a, b}, h2));
}
template <typename T> __device__ __forceinline__ v4s pack4(float a, float b, float c, float d) {
  typedef uint32_t u2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(v4s, (u2){pack2<T>(a, b), pack2<T>(c, d)});
}

// Partial slots are written through to the device's point of coherence
// (agent-scope relaxed atomic stores: global_store with sc1 on gfx950) rather
// than as non-temporal stores: the kernel-end L2 write-back before the merge
// kernel then has nothing of theirs left to do (3% shorter decode-attention
// launches at the e2e and tree shapes on MI355X).
__device__ __forceinline__ void store_wt(v4s* p, v4s v) {
  __hip_atomic_store(reinterpret_cast<unsigned long long*>(p), __builtin_bit_cast(unsigned long long, v),
                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_wt(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Four 16-bit values -> four floats (exact).
template <typename T> __device__ __forceinline__ v4f unpack4(v4s x);
template <> __device__ __forceinline__ v4f unpack4<bf16_t>(v4s x) {
  typedef uint32_t u2 __attribute__((ext_vector_type(2)));
  const u2 w = __builtin_bit_cast(u2, x);
  return v4f{__uint_as_float(w[0] << 16), __uint_as_float(w[0] & 0xffff0000u), __uint_as_float(w[1] << 16),
             __uint_as_float(w[1] & 0xffff0000u)};
}
template <> __device__ __forceinline__ v4f unpack4<f16_t>(v4s x) {
  typedef _Float16 h4 __attribute__((ext_vector_type(4)));
  return __builtin_convertvector(__builtin_bit_cast(h4, x), v4f);
}

// One wave's share of a 64-token tile: rows 16 rt + (0..15) against NSUB
// 16-token sub-tiles starting at kt / vt, for NMT head_dim tiles (voff).
// Online softmax state (m_run, l_run over this wave's tokens, o_acc) is
// updated in place; the rescale is skipped when no row's max rose.  P.V pairs
// two sub-tiles per v_mfma_f32_16x16x32: lane group lg holds tokens 4 lg..+3
// of both sub-tiles in the A (V^T) and B (P^T) operands alike, so the 32-wide
// contraction pairs the same tokens.
template <typename T, int NSUB, int NMT>
__device__ __forceinline__ void tile_compute(const unsigned char* kt, const unsigned char* vt, const v8s (&qf)[4],
                                             const uint32_t (&koff)[4], const uint32_t (&voff)[NMT], int tok_base,
                                             int vrow, int lg, float scale, float& m_run, float& l_run,
                                             v4f (&o_acc)[8]) {
  // all LDS operand reads first: the K fragments, then the V^T fragments
  // (independent of the scores, so their latency hides under the softmax)
  v8s kf[NSUB][4];
#pragma unroll
  for (int k = 0; k < NSUB; ++k)
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) kf[k][ks] = *reinterpret_cast<const v8s*>(kt + k * 4096 + koff[ks]);
  v4s vf[NMT][NSUB];
#pragma unroll
  for (int mt = 0; mt < NMT; ++mt)
#pragma unroll
    for (int k = 0; k < NSUB; ++k)
      vf[mt][k] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s_t)(vt + k * 4096 + voff[mt]));

  float x[NSUB][4];
#pragma unroll
  for (int k = 0; k < NSUB; ++k) {
    v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) acc = mfma_qk<T>(kf[k][ks], qf[ks], acc);
#pragma unroll
    for (int r = 0; r < 4; ++r) x[k][r] = acc[r] * scale;
  }
  // vrow: tokens of the tile this lane's row sees (the tile's valid tokens,
  // fewer under a causal limit)
  if (__builtin_amdgcn_ballot_w64(vrow < kTok) != 0) {
#pragma unroll
    for (int k = 0; k < NSUB; ++k)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (tok_base + k * 16 + 4 * lg + r >= vrow) x[k][r] = -INFINITY;
  }
  float mx = -INFINITY;
#pragma unroll
  for (int k = 0; k < NSUB; ++k)
#pragma unroll
    for (int r = 0; r < 4; ++r) mx = fmaxf(mx, x[k][r]);
  mx = rows4_max(mx);
  const float m_new = fmaxf(m_run, mx);
  const float msafe = (m_new == -INFINITY) ? 0.f : m_new;
  if (__builtin_amdgcn_ballot_w64(m_new > m_run) != 0) {
    const float alpha = __builtin_amdgcn_exp2f(m_run - msafe);
    l_run *= alpha;
#pragma unroll
    for (int mt = 0; mt < NMT; ++mt) o_acc[mt] *= alpha;
  }
  m_run = m_new;
  v4s pf[NSUB];
#pragma unroll
  for (int k = 0; k < NSUB; ++k) {
    float p[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      p[r] = __builtin_amdgcn_exp2f(x[k][r] - msafe);
      l_run += p[r];
    }
    pf[k] = pack4<T>(p[0], p[1], p[2], p[3]);
  }
  // O^T tiles: lane (lg, lc) supplied V[16 sub + 4 lg + lc/4][16 mt + 4 (lc%4) .. +3]
#pragma unroll
  for (int mt = 0; mt < NMT; ++mt) {
    v4f o = o_acc[mt];
    if constexpr (NSUB == 1) {
      o = mfma_pv<T>(vf[mt][0], pf[0], o);
    } else {
#pragma unroll
      for (int k = 0; k < NSUB; k += 2)
        o = mfma_qk<T>(__builtin_shufflevector(vf[mt][k], vf[mt][k + 1], 0, 1, 2, 3, 4, 5, 6, 7),
                       __builtin_shufflevector(pf[k], pf[k + 1], 0, 1, 2, 3, 4, 5, 6, 7), o);
    }
    o_acc[mt] = o;
  }
}

// Tokens of a tile (valid of them, starting at group token tile_tok) that
// row `row` of a segment sees when the segment's first query sees vis0 group
// tokens and query j (row / g) sees vis0 + j; kNoCausalS leaves valid.
__device__ __forceinline__ int row_limit(int valid, int vis0, int row, int g, int tile_tok) {
  return min(valid, max(0, vis0 + row / g - tile_tok));
}

// Wide wave roles: one wave's share of a 64-token tile for two 16-row MFMA
// tiles (32 rows) at once, so that every K and V^T fragment read from LDS
// feeds both (half the LDS reads per row of tile_compute).  qf[r], m_run[r],
// l_run[r] and o_acc[r] belong to row tile r; NSUB 16-token sub-tiles start
// at kt / vt (tokens tok_base ..); all 8 head_dim tiles.
template <typename T, int NSUB>
__device__ __forceinline__ void tile_compute_w(const unsigned char* kt, const unsigned char* vt,
                                               const v8s (&qf)[2][4], const uint32_t (&koff)[4],
                                               const uint32_t (&voff)[8], int tok_base, int valid, int lg,
                                               float scale, float (&m_run)[2], float (&l_run)[2],
                                               v4f (&o_acc)[2][8]) {
  v8s kf[NSUB][4];
#pragma unroll
  for (int k = 0; k < NSUB; ++k)
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) kf[k][ks] = *reinterpret_cast<const v8s*>(kt + k * 4096 + koff[ks]);
  v4s vf[8][NSUB];
#pragma unroll
  for (int mt = 0; mt < 8; ++mt)
#pragma unroll
    for (int k = 0; k < NSUB; ++k)
      vf[mt][k] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s_t)(vt + k * 4096 + voff[mt]));

  float x[2][NSUB][4];
#pragma unroll
  for (int r = 0; r < 2; ++r)
#pragma unroll
    for (int k = 0; k < NSUB; ++k) {
      v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) acc = mfma_qk<T>(kf[k][ks], qf[r][ks], acc);
#pragma unroll
      for (int i = 0; i < 4; ++i) x[r][k][i] = acc[i] * scale;
    }
  if (valid < tok_base + 16 * NSUB) {
#pragma unroll
    for (int k = 0; k < NSUB; ++k)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (tok_base + k * 16 + 4 * lg + i >= valid) {
          x[0][k][i] = -INFINITY;
          x[1][k][i] = -INFINITY;
        }
  }
  // row tile 0's softmax and P.V, then row tile 1's: row tile 1's softmax
  // (VALU) issues while row tile 0's P.V MFMAs execute
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    float mx = -INFINITY;
#pragma unroll
    for (int k = 0; k < NSUB; ++k)
#pragma unroll
      for (int i = 0; i < 4; ++i) mx = fmaxf(mx, x[r][k][i]);
    mx = rows4_max(mx);
    const float m_new = fmaxf(m_run[r], mx);
    const float msafe = (m_new == -INFINITY) ? 0.f : m_new;
    if (__builtin_amdgcn_ballot_w64(m_new > m_run[r]) != 0) {
      const float alpha = __builtin_amdgcn_exp2f(m_run[r] - msafe);
      l_run[r] *= alpha;
#pragma unroll
      for (int mt = 0; mt < 8; ++mt) o_acc[r][mt] *= alpha;
    }
    m_run[r] = m_new;
    v4s pf[NSUB];
#pragma unroll
    for (int k = 0; k < NSUB; ++k) {
      float p[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        p[i] = __builtin_amdgcn_exp2f(x[r][k][i] - msafe);
        l_run[r] += p[i];
      }
      pf[k] = pack4<T>(p[0], p[1], p[2], p[3]);
    }
#pragma unroll
    for (int mt = 0; mt < 8; ++mt) {
      v4f o = o_acc[r][mt];
      if constexpr (NSUB == 1) {
        o = mfma_pv<T>(vf[mt][0], pf[0], o);
      } else {
#pragma unroll
        for (int k = 0; k < NSUB; k += 2)
          o = mfma_qk<T>(__builtin_shufflevector(vf[mt][k], vf[mt][k + 1], 0, 1, 2, 3, 4, 5, 6, 7),
                         __builtin_shufflevector(pf[k], pf[k + 1], 0, 1, 2, 3, 4, 5, 6, 7), o);
      }
      o_acc[r][mt] = o;
    }
  }
}

// The 256-row wide roles' step: one wave's two 16-row MFMA tiles (32 rows)
// against a whole 64-token tile.  The scores of all 64 tokens come first (K
// fragments read in two 32-token halves to bound the registers), then one
// softmax step per row tile (one max reduction and one rescale check per
// tile), then P.V in two halves.  The scale enters the exponent as one FMA
// (p = 2^(s x - m) with m kept in the scaled domain), and the row sums l come
// from the MFMA pipe: a ones operand in place of V^T gives sum_t P[row][t] in
// every lane of the row (of the same 16-bit P that P.V uses), accumulated and
// rescaled like o.
template <typename T>
__device__ __forceinline__ void tile_compute_w64(const unsigned char* kt, const unsigned char* vt,
                                                 const v8s (&qf)[2][4], const uint32_t (&koff)[4],
                                                 const uint32_t (&voff)[8], int valid, int lg, float scale,
                                                 float (&m_run)[2], v4f (&l_acc)[2], v4f (&o_acc)[2][8]) {
  float x[2][4][4];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    v8s kf[2][4];
#pragma unroll
    for (int k = 0; k < 2; ++k)
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
        kf[k][ks] = *reinterpret_cast<const v8s*>(kt + (2 * h + k) * 4096 + koff[ks]);
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) acc = mfma_qk<T>(kf[k][ks], qf[r][ks], acc);
#pragma unroll
        for (int i = 0; i < 4; ++i) x[r][2 * h + k][i] = acc[i];
      }
  }
  if (valid < kTok) {
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (k * 16 + 4 * lg + i >= valid) {
          x[0][k][i] = -INFINITY;
          x[1][k][i] = -INFINITY;
        }
  }
  v4s pf[2][4];
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    float mx = -INFINITY;
#pragma unroll
    for (int k = 0; k < 4; ++k) mx = fmaxf(mx, fmaxf(fmaxf(x[r][k][0], x[r][k][1]), fmaxf(x[r][k][2], x[r][k][3])));
    mx = rows4_max(mx) * scale;                       // the scaled (log2-domain) max; scale > 0
    const float m_new = fmaxf(m_run[r], mx);
    const float msafe = (m_new == -INFINITY) ? 0.f : m_new;
    if (__builtin_amdgcn_ballot_w64(m_new > m_run[r]) != 0) {
      const float alpha = __builtin_amdgcn_exp2f(m_run[r] - msafe);
      l_acc[r] *= alpha;
#pragma unroll
      for (int mt = 0; mt < 8; ++mt) o_acc[r][mt] *= alpha;
    }
    m_run[r] = m_new;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      float p[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) p[i] = __builtin_amdgcn_exp2f(fmaf(x[r][k][i], scale, -msafe));
      pf[r][k] = pack4<T>(p[0], p[1], p[2], p[3]);
    }
  }
  constexpr short kOne = __is_same(T, bf16_t) ? (short)0x3F80 : (short)0x3C00;   // 1.0 in T
  const v8s ones = {kOne, kOne, kOne, kOne, kOne, kOne, kOne, kOne};
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    v4s vf[8][2];
#pragma unroll
    for (int mt = 0; mt < 8; ++mt)
#pragma unroll
      for (int k = 0; k < 2; ++k)
        vf[mt][k] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s_t)(vt + (2 * h + k) * 4096 + voff[mt]));
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const v8s pp = __builtin_shufflevector(pf[r][2 * h], pf[r][2 * h + 1], 0, 1, 2, 3, 4, 5, 6, 7);
      l_acc[r] = mfma_qk<T>(ones, pp, l_acc[r]);
#pragma unroll
      for (int mt = 0; mt < 8; ++mt)
        o_acc[r][mt] = mfma_qk<T>(__builtin_shufflevector(vf[mt][0], vf[mt][1], 0, 1, 2, 3, 4, 5, 6, 7), pp,
                                  o_acc[r][mt]);
    }
  }
}

}  // namespace stream
}  // namespace be

// Beam token selection for one decode step on gfx950.
//
// Reference: log_softmax + topk(2B) per row (beam.py:269-276) and the global
// top-B of VanillaBeamSearchStrategy.select_candidates with float64 scores and
// a stable sort (beam_strategy.py:433-488).  Floating-point contract (shared
// with the CPU restatement used as test oracle):
//   x'   = x                                           (temperature 1)
//   x'   = round_dtype(x * fl32(1 / T))                (BE_TEMP_RECIPROCAL: torch's
//          `logits / T` on a device tensor multiplies by the reciprocal of the
//          double temperature rounded to float)
//   x'   = round_dtype(x / T)                          (BE_TEMP_DIVIDE: correctly
//          rounded division, torch's `logits / T` on a CPU tensor)
//   m    = max_i x'_i
//   S    = sum_i exp(fl64(x'_i - m))                    (float64)
//   L    = fl32(ln S)
//   logp = round_dtype(fl32(fl32(x'_i - m) - L))
// Order: within a row (logp desc, index asc); in the pool (total desc,
// row*k + rank asc) with total = parent_score + (double)logp.
//
// Pass 1  grid (S, N): per segment max, float64 exp-sum and candidates -- the
//         positions whose x' reaches a threshold that >= k of them reach,
//         sorted -- with the largest x' below the threshold; the logits are
//         read once.
// Pass 2  grid (N):    the row's (m, L); the k best candidates by logp key,
//         ranked by merging the sorted segment lists; a row where an outside
//         value could tie the k-th is selected exactly over all its logits
//         instead.
// Pass 3  grid (R):    per request, the beam best of the row lists' pool by
//         merge ranks, emitted in pool-position order = grouped by row,
//         children in selection order.

#include <math.h>

#include <algorithm>
#include <atomic>
#include <mutex>

#include "common.h"

namespace be {

constexpr int kTopkThreads = 256;
constexpr int kMaxSegLen = 8192;     // logits per segment (32 per thread, in registers)
constexpr int kMaxSegs = 64;
constexpr int kMaxRowCand = 4096;    // candidates of one row (segments x cap), LDS in pass 2
constexpr int kMaxPool = 8192;       // rows x k of one request, LDS in pass 3
constexpr int kMaxPoolRows = 512;    // rows of one request
constexpr int kMaxK = 256;

// Candidate space per segment: 4k rounded up to a power of two, within [64, 256].
inline int topk_cap(int k) {
  int c = 64;
  while (c < 4 * k && c < 256) c *= 2;
  return c;
}

struct TopkGeom {
  int segs, seg_len;
};

static TopkGeom topk_geom(int n_rows, int vocab, int k) {
  int segs = (vocab + kMaxSegLen - 1) / kMaxSegLen;
  const int want = (512 + n_rows - 1) / n_rows;          // about two workgroups per CU
  if (want > segs) segs = want;
  const int by_k = (vocab + k - 1) / k;                   // every segment holds >= k elements
  if (segs > by_k) segs = by_k;
  if (segs > kMaxSegs) segs = kMaxSegs;
  if (segs * topk_cap(k) > kMaxRowCand) segs = kMaxRowCand / topk_cap(k);
  if (segs < 1) segs = 1;
  int seg_len = (vocab + segs - 1) / segs;
  seg_len = (seg_len + 7) & ~7;                           // 16-byte segment starts for 16-bit logits
  segs = (vocab + seg_len - 1) / seg_len;
  return TopkGeom{segs, seg_len};
}

// Bytes of the arrival counters at the start of the workspace: one u32 per
// row and one per request (at most 512 requests take the one-launch path).
// Counter words at the start of the workspace: one arrival counter per request
// (at most 512 requests take the two-launch path).
constexpr int kTopkCounterWords = 512;
inline int64_t topk_counter_bytes(int) { return ((int64_t)kTopkCounterWords * 4 + 255) / 256 * 256; }

// The hand-off from the rows pass's row workgroups to a request's pool pass
// (below) rests on how gfx942 / gfx950 treat agent-scope relaxed accesses:
// stores written through to the device's point of coherence (sc1), loads that
// read there, and in-order completion of a wave's vector memory operations
// before s_waitcnt vmcnt(0) returns.  Another target would need its own check.
#if defined(__HIP_DEVICE_COMPILE__) && !defined(__gfx950__) && !defined(__gfx942__)
#error "topk.hip's cross-workgroup hand-off is written for gfx942 / gfx950"
#endif

template <typename T>
__device__ __forceinline__ float load_logit(const T* p) { return to_f32(*p); }

template <typename T>
__device__ __forceinline__ float round_to(float x);
template <> __device__ __forceinline__ float round_to<float>(float x) { return x; }
template <> __device__ __forceinline__ float round_to<bf16_t>(float x) {
  return __uint_as_float(((uint32_t)f32_to_bf16_bits(x)) << 16);
}
template <> __device__ __forceinline__ float round_to<f16_t>(float x) { return (float)(_Float16)x; }

// Temperature scaling: tdiv == 0 multiplies by t (the float reciprocal of the
// temperature, computed on the host), tdiv == 1 divides by t (the temperature);
// t == 1 leaves the logits unchanged in both modes.
struct TempScale {
  float t;
  int tdiv;
};

template <typename T>
__device__ __forceinline__ float scaled(float x, TempScale ts) {
  if (ts.t == 1.0f) return x;
  return round_to<T>(ts.tdiv ? __fdiv_rn(x, ts.t) : __fmul_rn(x, ts.t));
}

constexpr int kPerThread = kMaxSegLen / kTopkThreads;   // logits per thread

// Position inside the segment of a thread's j-th logit: chunks of 16 bytes
// (8 bf16 / f16, 4 fp32), chunk c of thread t at c * 256 * V + t * V, so that
// one 16-byte load per chunk covers the segment's kMaxSegLen positions once.
template <typename T>
__device__ __forceinline__ int seg_pos(int j) {
  constexpr int V = 16 / (int)sizeof(T);
  return (j / V) * (kTopkThreads * V) + (int)threadIdx.x * V + (j % V);
}

// The thread's logits of one segment, temperature-scaled: 16-bit logits stay
// in their storage format, two to a register (x' is rounded to that format, so
// it is exact there), fp32 logits one to a register.  Positions >= n (past
// the segment) read as 0xffff (16-bit: a NaN, whose order key is 0) or -inf
// (fp32).
template <typename T>
struct SegVals {
  uint32_t w[kPerThread / 2];
  __device__ __forceinline__ float at(int j) const {
    const uint32_t u = w[j >> 1];
    if constexpr (sizeof(T) == 2 && __is_same(T, bf16_t)) {
      return __uint_as_float((j & 1) ? (u & 0xffff0000u) : (u << 16));
    } else {
      return (float)__builtin_bit_cast(_Float16, (uint16_t)((j & 1) ? (u >> 16) : (u & 0xffffu)));
    }
  }
};
template <>
struct SegVals<float> {
  float x[kPerThread];
  __device__ __forceinline__ float at(int j) const { return x[j]; }
};

template <typename T>
__device__ __forceinline__ uint16_t bits_of(float x);
template <> __device__ __forceinline__ uint16_t bits_of<bf16_t>(float x) { return f32_to_bf16_bits(x); }
template <> __device__ __forceinline__ uint16_t bits_of<f16_t>(float x) {
  return __builtin_bit_cast(uint16_t, (_Float16)x);
}

template <typename T>
__device__ __forceinline__ uint16_t raw_bits(const T* p) {
  return __builtin_bit_cast(uint16_t, *p);
}

// Loads n valid positions from seg (16-byte loads when the segment start is
// 16-byte aligned, uniform over the workgroup; else one load per logit).
constexpr uint16_t kPast16 = 0xffff;                   // past the segment: a negative NaN pattern, key 0

// The raw 16-bit logits of a segment (no temperature): only loads, so that a
// caller can issue them ahead of their use.
template <typename T>
__device__ __forceinline__ void load_raw16(const T* seg, int n, SegVals<T>& v) {
  constexpr int V = 8;
  const bool aligned = (reinterpret_cast<uintptr_t>(seg) & 15) == 0;
#pragma unroll
  for (int c = 0; c < kPerThread / V; ++c) {
    const int p0 = c * (kTopkThreads * V) + (int)threadIdx.x * V;
    if (aligned && p0 + V <= n) {
      const uint4 u = *reinterpret_cast<const uint4*>(seg + p0);
      v.w[c * 4 + 0] = u.x;
      v.w[c * 4 + 1] = u.y;
      v.w[c * 4 + 2] = u.z;
      v.w[c * 4 + 3] = u.w;
    } else {
#pragma unroll
      for (int e = 0; e < V; e += 2) {
        const uint32_t lo = p0 + e < n ? raw_bits(seg + p0 + e) : kPast16;
        const uint32_t hi = p0 + e + 1 < n ? raw_bits(seg + p0 + e + 1) : kPast16;
        v.w[c * 4 + e / 2] = lo | (hi << 16);
      }
    }
  }
}

// Temperature scaling of raw 16-bit logits in place (past-the-segment
// patterns stay).
template <typename T>
__device__ __forceinline__ void temp16(TempScale ts, SegVals<T>& v, int w0 = 0, int w1 = kPerThread / 2) {
  if (ts.t == 1.0f) return;
#pragma unroll
  for (int i = w0; i < w1; ++i) {
    const uint32_t u = v.w[i];
    const uint32_t lo = (u & 0xffffu) == kPast16 ? kPast16 : bits_of<T>(scaled<T>(v.at(2 * i), ts));
    const uint32_t hi = (u >> 16) == kPast16 ? kPast16 : bits_of<T>(scaled<T>(v.at(2 * i + 1), ts));
    v.w[i] = lo | (hi << 16);
  }
}

template <typename T>
__device__ __forceinline__ void load_vals(const T* seg, int n, TempScale ts, SegVals<T>& v) {
  constexpr int V = 8;                                 // 16-bit logits per 16 bytes
  constexpr uint16_t kPast = kPast16;
  const bool aligned = (reinterpret_cast<uintptr_t>(seg) & 15) == 0;
#pragma unroll
  for (int c = 0; c < kPerThread / V; ++c) {
    const int p0 = c * (kTopkThreads * V) + (int)threadIdx.x * V;
    if (aligned && p0 + V <= n) {
      const uint4 u = *reinterpret_cast<const uint4*>(seg + p0);
      v.w[c * 4 + 0] = u.x;
      v.w[c * 4 + 1] = u.y;
      v.w[c * 4 + 2] = u.z;
      v.w[c * 4 + 3] = u.w;
    } else {
#pragma unroll
      for (int e = 0; e < V; e += 2) {
        const uint32_t lo = p0 + e < n ? raw_bits(seg + p0 + e) : kPast;
        const uint32_t hi = p0 + e + 1 < n ? raw_bits(seg + p0 + e + 1) : kPast;
        v.w[c * 4 + e / 2] = lo | (hi << 16);
      }
    }
  }
  if (ts.t != 1.0f) {
#pragma unroll
    for (int i = 0; i < kPerThread / 2; ++i) {
      const uint32_t u = v.w[i];
      const uint32_t lo = (u & 0xffffu) == kPast ? kPast : bits_of<T>(scaled<T>(v.at(2 * i), ts));
      const uint32_t hi = (u >> 16) == kPast ? kPast : bits_of<T>(scaled<T>(v.at(2 * i + 1), ts));
      v.w[i] = lo | (hi << 16);
    }
  }
}
template <>
__device__ __forceinline__ void load_vals<float>(const float* seg, int n, TempScale ts, SegVals<float>& v) {
  constexpr int V = 4;
  const bool aligned = (reinterpret_cast<uintptr_t>(seg) & 15) == 0;
#pragma unroll
  for (int c = 0; c < kPerThread / V; ++c) {
    const int p0 = c * (kTopkThreads * V) + (int)threadIdx.x * V;
    if (aligned && p0 + V <= n) {
      const float4 u = *reinterpret_cast<const float4*>(seg + p0);
      v.x[c * 4 + 0] = scaled<float>(u.x, ts);
      v.x[c * 4 + 1] = scaled<float>(u.y, ts);
      v.x[c * 4 + 2] = scaled<float>(u.z, ts);
      v.x[c * 4 + 3] = scaled<float>(u.w, ts);
    } else {
#pragma unroll
      for (int e = 0; e < V; ++e) v.x[c * 4 + e] = p0 + e < n ? scaled<float>(seg[p0 + e], ts) : -INFINITY;
    }
  }
}

// ---------------------------------------------------------------- DPP wave scans
// Inclusive scans over the 64 lanes of a wave on the VALU (no LDS): row_shr 1,
// 2, 4, 8 within each 16-lane row, then row_bcast:15 and row_bcast:31 carry the
// row totals upward; lane 63 ends with the whole wave's value.
template <int CTRL, int ROWS, bool ZERO>
__device__ __forceinline__ uint32_t dpp(uint32_t old, uint32_t src) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)old, (int)src, CTRL, ROWS, 0xf, ZERO);
}

__device__ __forceinline__ int wave_scan_add(int x) {
  x += (int)dpp<0x111, 0xf, true>(0, x);
  x += (int)dpp<0x112, 0xf, true>(0, x);
  x += (int)dpp<0x114, 0xf, true>(0, x);
  x += (int)dpp<0x118, 0xf, true>(0, x);
  x += (int)dpp<0x142, 0xa, false>(0, x);
  x += (int)dpp<0x143, 0xc, false>(0, x);
  return x;
}

__device__ __forceinline__ uint32_t wave_scan_max(uint32_t x) {
  x = max(x, dpp<0x111, 0xf, true>(0, x));
  x = max(x, dpp<0x112, 0xf, true>(0, x));
  x = max(x, dpp<0x114, 0xf, true>(0, x));
  x = max(x, dpp<0x118, 0xf, true>(0, x));
  x = max(x, dpp<0x142, 0xa, false>(0, x));
  x = max(x, dpp<0x143, 0xc, false>(0, x));
  return x;
}

template <int CTRL, int ROWS, bool ZERO>
__device__ __forceinline__ double dpp_f64(double src) {
  const uint64_t u = (uint64_t)__double_as_longlong(src);
  const uint32_t lo = dpp<CTRL, ROWS, ZERO>(0, (uint32_t)u);
  const uint32_t hi = dpp<CTRL, ROWS, ZERO>(0, (uint32_t)(u >> 32));
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

// A fixed order of additions: the sum does not depend on timing.
__device__ __forceinline__ double wave_scan_add_f64(double x) {
  x += dpp_f64<0x111, 0xf, true>(x);
  x += dpp_f64<0x112, 0xf, true>(x);
  x += dpp_f64<0x114, 0xf, true>(x);
  x += dpp_f64<0x118, 0xf, true>(x);
  x += dpp_f64<0x142, 0xa, false>(x);
  x += dpp_f64<0x143, 0xc, false>(x);
  return x;
}

__device__ __forceinline__ uint32_t lane63(uint32_t x) { return (uint32_t)__builtin_amdgcn_readlane((int)x, 63); }

__device__ __forceinline__ uint32_t fkey(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ uint64_t dkey(double f) {
  const uint64_t u = (uint64_t)__double_as_longlong(f);
  return (u & 0x8000000000000000ull) ? ~u : (u | 0x8000000000000000ull);
}

// ---------------------------------------------------------------- 16-bit keys
typedef unsigned short v2u16 __attribute__((ext_vector_type(2)));
typedef short v2i16 __attribute__((ext_vector_type(2)));

// Order-preserving 16-bit keys of two packed 16-bit floats (bf16 or f16 bit
// patterns): negative values get their bits inverted, the others the sign bit
// set.  0xffff (a negative NaN pattern: positions past the segment) maps to 0,
// below every other key.
__device__ __forceinline__ uint32_t key16x2(uint32_t u) {
  const v2i16 sgn = __builtin_bit_cast(v2i16, u) >> (v2i16){15, 15};   // 0xffff where negative
  return u ^ (__builtin_bit_cast(uint32_t, sgn) | 0x80008000u);
}

// The 32-bit key (fkey of the float value) of the 16-bit value with key k16.
template <typename T>
__device__ __forceinline__ uint32_t key32_of16(uint32_t k16) {
  const uint16_t raw = (uint16_t)((k16 & 0x8000u) ? (k16 ^ 0x8000u) : (~k16 & 0xffffu));
  return fkey(to_f32(__builtin_bit_cast(T, raw)));
}

// Block-wide inclusive suffix sum (over threads >= tid) of one int per
// thread of an NT-thread block: shuffles inside each wave, then the wave
// totals through LDS (two barriers instead of a barrier pair per doubling
// step).  tot holds NT / 64 ints.
template <int NT = kTopkThreads>
__device__ __forceinline__ int block_suffix_sum(int v, int* tot) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int u = __shfl_down(v, o, 64);
    if (lane + o < 64) v += u;
  }
  if (lane == 0) tot[w] = v;
  __syncthreads();
  for (int x = w + 1; x < NT / 64; ++x) v += tot[x];
  __syncthreads();
  return v;
}
// Row max m and L = fl32(ln S) from the segment statistics, once per
// workgroup: wave 0 takes one segment per lane (S_s exp(m_s - m) in
// parallel), lane 0 adds the terms in segment order (a fixed float64 sum).
__device__ __forceinline__ void row_norm_block(const float* seg_max, const double* seg_sum, int r, int segs,
                                               float& m, float& L, double* terms, float* mL) {
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    const float ms = lane < segs ? seg_max[(int64_t)r * segs + lane] : -INFINITY;
    const float mm = wave_max(ms);
    terms[lane] = lane < segs ? seg_sum[(int64_t)r * segs + lane] * exp((double)ms - (double)mm) : 0.0;
    if (lane == 0) {
      double S = 0.0;
      for (int s = 0; s < segs; ++s) S += terms[s];
      mL[0] = mm;
      mL[1] = (float)log(S);
    }
  }
  __syncthreads();
  m = mL[0];
  L = mL[1];
}

template <typename T>
__device__ __forceinline__ float logp_of(float xs, float m, float L) {
  return round_to<T>(__fsub_rn(__fsub_rn(xs, m), L));
}

// ---------------------------------------------------------------- wave sort
__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
  const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)v, m, 64);
  const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), m, 64);
  return ((uint64_t)hi << 32) | lo;
}

// Wave-wide bitonic sort, descending, of NPL * 64 values: item q = e * 64 + lane
// lives in v[e] of that lane.  Partners 64 or more items apart are in the
// same lane (a register exchange), nearer ones in another lane (a shuffle).
template <int NPL>
__device__ __forceinline__ void wave_sort_desc_u64(uint64_t (&v)[NPL]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int size = 2; size <= 64 * NPL; size <<= 1) {
#pragma unroll
    for (int j = size >> 1; j > 0; j >>= 1) {
      if (j >= 64) {
        const int je = j >> 6;
#pragma unroll
        for (int e = 0; e < NPL; ++e) {
          if ((e & je) == 0) {
            // q & size does not depend on the lane: size > j >= 64
            const bool first = ((e * 64) & size) == 0;
            const uint64_t a = v[e], b = v[e | je];
            const uint64_t hi = a > b ? a : b, lo = a > b ? b : a;
            v[e] = first ? hi : lo;
            v[e | je] = first ? lo : hi;
          }
        }
      } else {
#pragma unroll
        for (int e = 0; e < NPL; ++e) {
          const uint64_t p = shfl_xor_u64(v[e], j);
          const int q = e * 64 + lane;
          const bool lower = (q & j) == 0, first = (q & size) == 0;
          // descending blocks where first: the lower item keeps the larger value
          v[e] = (lower == first) ? (v[e] > p ? v[e] : p) : (v[e] < p ? v[e] : p);
        }
      }
    }
  }
}

// ---------------------------------------------------------------- float64 exp
// e^d for d <= 0, accurate to about one ulp, without branches: Tang's
// table-driven method.  k = rint(d 64 / ln 2), r = d - k ln2/64 (Cody-Waite,
// hi part of 36 bits so k * hi is exact), e^r - 1 by its degree-5 Taylor
// polynomial (|r| <= ln2/128: the first omitted term, r^6/720, is below
// 4e-17), times 2^((k mod 64) / 64) from a 64-entry table and 2^floor(k / 64).
// rint comes from adding 1.5 * 2^52 (k is then the low word of the sum) and
// 2^floor(k / 64) from adding floor(k / 64) to the table entry's exponent, so
// no rounding, conversion or ldexp instruction is needed.  d is clamped to
// -708 first (fmax also maps NaN there), which keeps that exponent normal:
// -inf, NaN and anything below give e^-708, nothing against the sums of at
// least 1 these terms go into.
constexpr double kInvLn2x64 = 0x1.71547652b82fep+6;
constexpr double kLn2By64Hi = 0x1.62e42fefa0000p-7;
constexpr double kLn2By64Lo = 0x1.cf79abc9e3b3ap-46;
constexpr double kRoundShift = 0x1.8p52;

__device__ __forceinline__ void exp_table_init(double* tab) {
  if (threadIdx.x < 64) tab[threadIdx.x] = exp2((double)threadIdx.x / 64.0);
}

__device__ __forceinline__ double exp_neg(double d, const double* tab) {
  const double dc = fmax(d, -708.0);
  const double sh = fma(dc, kInvLn2x64, kRoundShift);
  const int k = (int)(uint32_t)(uint64_t)__double_as_longlong(sh);
  const double kf = sh - kRoundShift;
  double r = fma(-kf, kLn2By64Hi, dc);
  r = fma(-kf, kLn2By64Lo, r);
  double p = fma(r, 1.0 / 120.0, 1.0 / 24.0);
  p = fma(r, p, 1.0 / 6.0);
  p = fma(r, p, 0.5);
  p = fma(r, p, 1.0);
  p *= r;                                           // e^r - 1
  const uint64_t tb = (uint64_t)__double_as_longlong(tab[k & 63]);
  const uint32_t hi = (uint32_t)(tb >> 32) + ((uint32_t)(k >> 6) << 20);
  const double t = __longlong_as_double((long long)(((uint64_t)hi << 32) | (uint32_t)tb));
  return fma(t, p, t);
}

// ---------------------------------------------------------------- pass 1
constexpr int kMaxCap = 256;

// The segment's candidates (lc[0, total), composite keys) sorted descending by
// wave 0 and written to out.
template <int NPL>
__device__ __forceinline__ void sort_out_candidates(const uint64_t* lc, int total, uint64_t* out) {
  const int lane = threadIdx.x & 63;
  uint64_t v[NPL];
#pragma unroll
  for (int e = 0; e < NPL; ++e) v[e] = e * 64 + lane < total ? lc[e * 64 + lane] : 0ull;
  wave_sort_desc_u64<NPL>(v);
#pragma unroll
  for (int e = 0; e < NPL; ++e)
    if (e * 64 + lane < total) out[e * 64 + lane] = v[e];
}

// Per (segment, row): the segment max m_s and S_s = sum exp(x' - m_s) in
// float64 (x' the temperature-scaled logits; logits are read once), and the
// segment's candidates: every position whose x' reaches a threshold tau that
// at least k positions reach (the smallest of the four waves' ceil(k/4)-th
// largest per-thread maximum, found bit by bit with ballots), as composite
// keys (order-preserving key of x') << 32 | ~(vocabulary index), sorted
// descending (x' descending, index ascending), plus the largest key below tau
// (0 if none).  More than `cap` candidates is flagged (count -1).  logp is
// monotone in x', so a row's best logp values are among its segments'
// candidates unless a segment's largest outside value rounds to the same logp
// as the row's k-th candidate -- pass 2 checks exactly that.
//
// Waves per SIMD the register budget allows: the kernel is latency-bound, so
// more resident workgroups hide more of it.
constexpr int kCandWavesPerSimd = 8;

// One barrier exchanges the waves' maxima, float64 sums (each against its
// wave's max) and thresholds; wave reductions and scans run on DPP; each wave
// takes its candidates' LDS slots with one atomic add (their order there does
// not matter: wave 0 sorts them).
// The segment's float64 sum from the waves' sums (each against its wave's
// max), its candidates sorted out by wave 0, and its statistics.
__device__ __forceinline__ void finish_segment(const uint64_t* lc, int total, int cap, float m, const float* wmax,
                                               const double* wsum, const double* tab, uint32_t bound, int64_t rs,
                                               float* seg_max, double* seg_sum, int* seg_cnt, uint32_t* seg_bound,
                                               uint64_t* cand) {
  if (total <= cap && threadIdx.x < 64) {
    uint64_t* out = cand + rs * cap;
    if (total <= 64) sort_out_candidates<1>(lc, total, out);
    else if (total <= 128) sort_out_candidates<2>(lc, total, out);
    else sort_out_candidates<4>(lc, total, out);
  }
  if (threadIdx.x == 0) {
    // the waves' sums rescaled to the segment max, in wave order
    double sum = 0.0;
    for (int q = 0; q < 4; ++q) sum += wsum[q] * exp_neg((double)wmax[q] - (double)m, tab);
    seg_max[rs] = m;
    seg_sum[rs] = sum;
    seg_cnt[rs] = total <= cap ? total : -1;
    seg_bound[rs] = bound;
  }
}

// fp32 logits: 32-bit keys (one logit to a register: four waves per SIMD
// leave it room without spills).
template <typename T>
__global__ __launch_bounds__(kTopkThreads, 4) void topk_cand_kernel(const T* logits, int64_t row_stride, int vocab,
                                                                int seg_len, TempScale ts, int k, int cap,
                                                                float* seg_max, double* seg_sum, int* seg_cnt,
                                                                uint32_t* seg_bound, uint64_t* cand) {
  __shared__ double tab[64];
  __shared__ float wmax[4];
  __shared__ double wsum[4];
  __shared__ uint32_t wtau[4];
  __shared__ uint32_t wbelow[4];
  __shared__ int ncand;
  __shared__ uint64_t lc[kMaxCap];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int s = blockIdx.x, r = blockIdx.y, segs = gridDim.x;
  const T* row = logits + (int64_t)r * row_stride;
  const int b = s * seg_len, n = min(vocab, b + seg_len) - b;
  exp_table_init(tab);
  if (tid == 0) ncand = 0;
  SegVals<T> x;
  load_vals<T>(row + b, n, ts, x);
  // key 0 marks positions past the segment (valid keys are >= fkey(-inf) > 0)
  auto key_at = [&](int j) -> uint32_t { return seg_pos<T>(j) < n ? fkey(x.at(j)) : 0u; };
  uint32_t kmax = 0;
#pragma unroll
  for (int j = 0; j < kPerThread; ++j) kmax = max(kmax, key_at(j));
  // the thread max: -inf when the thread holds no position or only -inf
  const float mt = kmax > fkey(-INFINITY) ? __uint_as_float((kmax & 0x80000000u) ? (kmax & 0x7fffffffu) : ~kmax)
                                          : -INFINITY;
  // the wave's kw-th largest per-thread maximum, bit by bit
  const int kw = (k + 3) >> 2;                         // <= 64
  uint32_t pref = 0;
  for (int bit = 31; bit >= 0; --bit) {
    const uint32_t c = pref | (1u << bit);
    if (__popcll(__builtin_amdgcn_ballot_w64(kmax >= c)) >= kw) pref = c;
  }
  const uint32_t kwave = lane63(wave_scan_max(kmax));  // key of the wave max
  __syncthreads();                                     // the exp table, ncand
  // float64 sum against the thread's own max, then against the wave's
  const double md = (double)mt;
  double acc = 0.0;
#pragma unroll
  for (int j = 0; j < kPerThread; ++j) acc += exp_neg((double)x.at(j) - md, tab);
  const float mw = kwave > fkey(-INFINITY)
                       ? __uint_as_float((kwave & 0x80000000u) ? (kwave & 0x7fffffffu) : ~kwave)
                       : -INFINITY;
  acc = mt == -INFINITY ? 0.0 : acc * exp_neg(md - (double)mw, tab);
  acc = wave_scan_add_f64(acc);
  if (lane == 63) {
    wmax[w] = mw;
    wsum[w] = acc;
    wtau[w] = pref;
  }
  __syncthreads();
  const float m = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
  const uint32_t tau = max(1u, min(min(wtau[0], wtau[1]), min(wtau[2], wtau[3])));
  int mine = 0;
  uint32_t below = 0;
#pragma unroll
  for (int j = 0; j < kPerThread; ++j) {
    const uint32_t key = key_at(j);
    mine += key >= tau ? 1 : 0;
    below = max(below, key < tau ? key : 0u);
  }
  const int incl = wave_scan_add(mine);
  int wbase = 0;
  if (lane == 63) wbase = atomicAdd(&ncand, incl);
  int at = (int)lane63((uint32_t)wbase) + incl - mine;
  if (mine > 0) {
#pragma unroll
    for (int j = 0; j < kPerThread; ++j) {
      const uint32_t key = key_at(j);
      if (key >= tau) {
        if (at < cap) lc[at] = ((uint64_t)key << 32) | (uint32_t)~(uint32_t)(b + seg_pos<T>(j));
        ++at;
      }
    }
  }
  below = wave_scan_max(below);
  if (lane == 63) wbelow[w] = below;
  __syncthreads();
  finish_segment(lc, ncand, cap, m, wmax, wsum, tab, max(max(wbelow[0], wbelow[1]), max(wbelow[2], wbelow[3])),
                 (int64_t)r * segs + s, seg_max, seg_sum, seg_cnt, seg_bound, cand);
}

// 16-bit logits: packed 16-bit order keys, two to a register (packed u16 max,
// saturating subtract and min count and compare two logits per instruction),
// a 16-bit threshold search, and as the boundary key the value just below the
// threshold (an upper bound of every outside value).
template <typename T>
__global__ __launch_bounds__(kTopkThreads, kCandWavesPerSimd) void topk_cand16_kernel(const T* logits, int64_t row_stride, int vocab,
                                                                  int seg_len, TempScale ts, int k, int cap,
                                                                  float* seg_max, double* seg_sum, int* seg_cnt,
                                                                  uint32_t* seg_bound, uint64_t* cand) {
  __shared__ double tab[64];
  __shared__ float wmax[4];
  __shared__ double wsum[4];
  __shared__ uint32_t wtau[4];
  __shared__ int ncand;
  __shared__ uint64_t lc[kMaxCap];
  constexpr int kWords = kPerThread / 2;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int s = blockIdx.x, r = blockIdx.y, segs = gridDim.x;
  const T* row = logits + (int64_t)r * row_stride;
  const int b = s * seg_len, n = min(vocab, b + seg_len) - b;
  exp_table_init(tab);
  if (tid == 0) ncand = 0;
  SegVals<T> x;
  load_vals<T>(row + b, n, ts, x);
  uint32_t kp[kWords];
  v2u16 km2 = {0, 0};
#pragma unroll
  for (int i = 0; i < kWords; ++i) {
    kp[i] = key16x2(x.w[i]);
    km2 = __builtin_elementwise_max(km2, __builtin_bit_cast(v2u16, kp[i]));
  }
  const uint32_t kmax = max((uint32_t)km2.x, (uint32_t)km2.y);
  const uint32_t kninf = key16x2(__is_same(T, bf16_t) ? 0xff80u : 0xfc00u) & 0xffffu;   // key of -inf
  auto value_of = [&](uint32_t k16) -> float {
    return k16 > kninf ? to_f32(__builtin_bit_cast(T, (uint16_t)((k16 & 0x8000u) ? (k16 ^ 0x8000u) : (~k16 & 0xffffu))))
                       : -INFINITY;
  };
  const float mt = value_of(kmax);
  // the wave's kw-th largest per-thread maximum, bit by bit
  const int kw = (k + 3) >> 2;                         // <= 64
  uint32_t pref = 0;
  for (int bit = 15; bit >= 0; --bit) {
    const uint32_t c = pref | (1u << bit);
    if (__popcll(__builtin_amdgcn_ballot_w64(kmax >= c)) >= kw) pref = c;
  }
  const float mw = value_of(lane63(wave_scan_max(kmax)));
  __syncthreads();                                     // the exp table, ncand
  // float64 sum against the thread's own max, then against the wave's
  // (positions past the segment read as NaN: exp_neg gives 0)
  const double md = (double)mt;
  double acc = 0.0;
#pragma unroll
  for (int j = 0; j < kPerThread; ++j) acc += exp_neg((double)x.at(j) - md, tab);
  acc = mt == -INFINITY ? 0.0 : acc * exp_neg(md - (double)mw, tab);
  acc = wave_scan_add_f64(acc);
  if (lane == 63) {
    wmax[w] = mw;
    wsum[w] = acc;
    wtau[w] = pref;
  }
  __syncthreads();
  const float m = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
  const uint32_t tau = max(1u, min(min(wtau[0], wtau[1]), min(wtau[2], wtau[3])));
  // count of keys >= tau: min(sat(key - (tau - 1)), 1) per half
  const v2u16 t1 = {(unsigned short)(tau - 1), (unsigned short)(tau - 1)};
  const v2u16 one = {1, 1};
  v2u16 c2 = {0, 0};
#pragma unroll
  for (int i = 0; i < kWords; ++i)
    c2 += __builtin_elementwise_min(__builtin_elementwise_sub_sat(__builtin_bit_cast(v2u16, kp[i]), t1), one);
  const int mine = (int)c2.x + (int)c2.y;
  const int incl = wave_scan_add(mine);
  int wbase = 0;
  if (lane == 63) wbase = atomicAdd(&ncand, incl);
  int at = (int)lane63((uint32_t)wbase) + incl - mine;
  if (mine > 0) {
#pragma unroll
    for (int i = 0; i < kWords; ++i) {
      const uint32_t lo = kp[i] & 0xffffu, hi = kp[i] >> 16;
      if (max(lo, hi) >= tau) {
        if (lo >= tau) {
          if (at < cap) lc[at] = ((uint64_t)key32_of16<T>(lo) << 32) | (uint32_t)~(uint32_t)(b + seg_pos<T>(2 * i));
          ++at;
        }
        if (hi >= tau) {
          if (at < cap)
            lc[at] = ((uint64_t)key32_of16<T>(hi) << 32) | (uint32_t)~(uint32_t)(b + seg_pos<T>(2 * i + 1));
          ++at;
        }
      }
    }
  }
  __syncthreads();
  finish_segment(lc, ncand, cap, m, wmax, wsum, tab, tau > 1 ? key32_of16<T>(tau - 1) : 0u,
                 (int64_t)r * segs + s, seg_max, seg_sum, seg_cnt, seg_bound, cand);
}

// ---------------------------------------------------------------- selection helper
// The k best of n items by (key desc, idx asc), keys and vocabulary indices
// given by key_of(i) / idx_of(i), i < n (n >= k): a radix select of the k-th
// largest key (4 passes of 8 bits), every item above it, and among the items
// equal to it the lowest indices (a second radix select, over inverted
// indices, only when the ties exceed what is needed).  Writes the k chosen
// (key, idx) pairs to out_key / out_idx (LDS, unordered).  All threads call it.
template <int NT = kTopkThreads, typename KeyF, typename IdxF>
__device__ void select_k(KeyF key_of, IdxF idx_of, int n, int k, uint32_t* out_key, int32_t* out_idx,
                         int* hist /*4*256*/, int* suf /*257*/, int* misc /*4 + NT/64*/) {
  const int tid = threadIdx.x, w = tid >> 6;
  auto radix = [&](auto val_of, auto live, int want, uint32_t& prefix_out) -> int {
    // returns how many of the `want` remain at the selected value prefix_out
    uint32_t prefix = 0, mask = 0;
    int krem = want;
    for (int shift = 24; shift >= 0; shift -= 8) {
      for (int i = tid; i < 4 * 256; i += NT) hist[i] = 0;
      __syncthreads();
      for (int i = tid; i < n; i += NT) {
        if (!live(i)) continue;
        const uint32_t v = val_of(i);
        if ((v & mask) == prefix) atomicAdd(&hist[(w & 3) * 256 + (int)((v >> shift) & 255u)], 1);
      }
      __syncthreads();
      const int hv = tid < 256 ? hist[tid] + hist[256 + tid] + hist[512 + tid] + hist[768 + tid] : 0;
      const int sv = block_suffix_sum<NT>(hv, misc + 4);
      if (tid < 256) suf[tid] = sv;
      if (tid == 0) suf[256] = 0;
      __syncthreads();
      if (tid < 256 && suf[tid] >= krem && suf[tid + 1] < krem) {
        misc[0] = tid;
        misc[1] = suf[tid + 1];
      }
      __syncthreads();
      krem -= misc[1];
      prefix |= ((uint32_t)misc[0]) << shift;
      mask |= 255u << shift;
      __syncthreads();
    }
    prefix_out = prefix;
    return krem;
  };
  uint32_t T;
  const int krem = radix(key_of, [](int) { return true; }, k, T);
  // items above T, and the count of ties
  if (tid == 0) {
    misc[2] = 0;
    misc[3] = 0;
  }
  __syncthreads();
  for (int i = tid; i < n; i += NT) {
    const uint32_t v = key_of(i);
    if (v > T) {
      const int at = atomicAdd(&misc[2], 1);
      out_key[at] = v;
      out_idx[at] = idx_of(i);
    } else if (v == T) {
      atomicAdd(&misc[3], 1);
    }
  }
  __syncthreads();
  const int ngt = k - krem, nties = misc[3];
  if (nties == krem) {
    if (tid == 0) misc[2] = ngt;
    __syncthreads();
    for (int i = tid; i < n; i += NT)
      if (key_of(i) == T) {
        const int at = atomicAdd(&misc[2], 1);
        out_key[at] = T;
        out_idx[at] = idx_of(i);
      }
  } else {
    // the krem lowest indices among the ties: largest inverted index
    uint32_t I;
    radix([&](int i) { return 0xffffffffu - (uint32_t)idx_of(i); }, [&](int i) { return key_of(i) == T; }, krem, I);
    if (tid == 0) misc[2] = ngt;
    __syncthreads();
    for (int i = tid; i < n; i += NT)
      if (key_of(i) == T && 0xffffffffu - (uint32_t)idx_of(i) >= I) {
        const int at = atomicAdd(&misc[2], 1);
        out_key[at] = T;
        out_idx[at] = idx_of(i);
      }
  }
  __syncthreads();
}

// ---------------------------------------------------------------- pass 2
// Per row: the row's (m, L) from the segment statistics, then the k best
// candidates by (logp desc, index asc) from the segments' lists (sorted by
// x' desc, index asc):
//  1. the row's k best by x' -- every list entry is ranked by counting, in
//     each other list, the entries above it (binary searches over the first
//     k entries, sixteen lists at a time, with selects rather than branches
//     so that their LDS reads overlap), list positions in chunks of 16 until
//     no list has a further entry of rank < k;
//  2. logp is monotone in x', so the k-th logp is the logp of the k-th x';
//     the entries above it are selected, and from its tie group (every
//     candidate with that logp, gathered wave by wave over the lists) the
//     ones of lowest index;
//  3. the k selected are ordered by (logp desc, index asc) by counting.
// The candidates hold the row's k best unless a segment overflowed its
// candidate space, the tie group overflows its LDS array, or a segment's
// outside values (all at most its boundary key) reach the k-th logp; then the
// row is selected exactly over all its logits.
constexpr int kSlotsPerThread = kMaxRowCand / kTopkThreads;
constexpr int kMaxTie = 512;

template <typename T>
__global__ __launch_bounds__(kTopkThreads) void topk_row_kernel(const T* logits, int64_t row_stride, int vocab,
                                                               TempScale ts, int segs, int k, int cap,
                                                               const float* seg_max, const double* seg_sum,
                                                               const int* seg_cnt, const uint32_t* seg_bound,
                                                               const uint64_t* cand, float* row_vals,
                                                               int32_t* row_idx) {
  __shared__ uint64_t la[kMaxRowCand];                 // x' composite keys, list after list
  __shared__ uint64_t bx[kMaxK];                       // the k best by x' composite, in order
  __shared__ uint64_t tg[kMaxTie];                     // the tie group (logp composite keys)
  __shared__ uint64_t fin[kMaxK];                      // the k selected (logp composite keys)
  __shared__ uint32_t skey[kMaxK];
  __shared__ int32_t sidx[kMaxK];
  __shared__ int hist[4 * 256];
  __shared__ int suf[257];
  __shared__ int misc[8];
  __shared__ double terms[64];
  __shared__ float mL[2];
  __shared__ int off[kMaxSegs + 1];
  __shared__ int more[kMaxK / 16];
  __shared__ int flag, ntie, nfin;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, r = blockIdx.x;
  const int64_t base = (int64_t)r * segs;
  const int lcap = __ffs(cap) - 1;                     // cap is a power of two
  const int nslots = segs << lcap;
  // the row's candidate slots (segs lists of cap), loaded at once; slots past
  // a list's count hold stale words and are not used
  const uint64_t* blk = cand + base * cap;
  uint64_t v[kSlotsPerThread];
#pragma unroll
  for (int u = 0; u < kSlotsPerThread; ++u)
    if (u * kTopkThreads < nslots) v[u] = blk[min(u * kTopkThreads + tid, nslots - 1)];
  if (tid < kMaxK / 16) more[tid] = 0;
  if (tid == 0) {
    ntie = 0;
    nfin = 0;
  }
  if (tid < 64) {
    const int c = tid < segs ? seg_cnt[base + tid] : 0;
    int incl = c < 0 ? 0 : c;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int u = __shfl_up(incl, o, 64);
      if (tid >= o) incl += u;
    }
    if (tid < segs) off[tid + 1] = incl;
    if (tid == 0) off[0] = 0;
    const bool over = __builtin_amdgcn_ballot_w64(c < 0) != 0;
    if (tid == 0) flag = over ? 1 : 0;
  }
  float m, L;
  row_norm_block(seg_max, seg_sum, r, segs, m, L, terms, mL);   // (its barrier publishes the above)
  auto key_of_x = [&](uint32_t xk) -> uint32_t {       // x' key -> logp key
    const uint32_t u = (xk & 0x80000000u) ? (xk & 0x7fffffffu) : ~xk;
    return fkey(logp_of<T>(__uint_as_float(u), m, L));
  };
  bool exact = flag != 0;
  if (!exact) {
#pragma unroll
    for (int u = 0; u < kSlotsPerThread; ++u) {
      const int f = u * kTopkThreads + tid, sg = f >> lcap, p = f & (cap - 1);
      if (f < nslots) {
        const int lo = off[sg];
        if (p < off[sg + 1] - lo) la[lo + p] = v[u];
      }
    }
    __syncthreads();
    // 1. the k best by x'
    int top = 1;
    while (top * 2 <= k) top *= 2;
    for (int c0 = 0; c0 < k; c0 += 16) {
      for (int f = tid; f < segs * 16; f += kTopkThreads) {
        const int sg = f >> 4, p = c0 + (f & 15);
        const int lo = off[sg], len = off[sg + 1] - lo;
        if (p >= len) continue;
        const uint64_t key = la[lo + p];
        int rank = p;
        for (int l0 = 0; l0 < segs && rank < k; l0 += 16) {
          int pos[16], bs[16], ln[16];
#pragma unroll
          for (int u = 0; u < 16; ++u) {
            const int l = l0 + u;
            const bool use = (l < segs) & (l != sg);
            const int o0 = off[min(l, segs)], o1 = off[min(l + 1, segs)];
            bs[u] = use ? o0 : 0;
            ln[u] = use ? min(o1 - o0, k) : 0;
            pos[u] = 0;
          }
          for (int step = top; step > 0; step >>= 1) {
            uint64_t y[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) y[u] = la[max(bs[u] + min(pos[u] + step, ln[u]) - 1, 0)];
            // the sixteen reads are issued before any compare waits for one
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int u = 0; u < 16; ++u) {
              const int c = pos[u] + step;
              // bitwise & keeps the choice a select (a short-circuit && would let
              // the compiler sink the read under a branch)
              pos[u] = ((c <= ln[u]) & (y[u] > key)) ? c : pos[u];
            }
          }
#pragma unroll
          for (int u = 0; u < 16; ++u) rank += pos[u];
        }
        if (rank < k) {
          bx[rank] = key;
          if ((f & 15) == 15 && p + 1 < len) more[c0 >> 4] = 1;
        }
      }
      __syncthreads();
      if (!more[c0 >> 4]) break;
    }
    // 2. the k-th logp; the entries above it, and its tie group
    const uint32_t kth = key_of_x((uint32_t)(bx[k - 1] >> 32));
    for (int i = tid; i < k; i += kTopkThreads) {
      const uint64_t x = bx[i];
      const uint32_t lk = key_of_x((uint32_t)(x >> 32));
      if (lk > kth) fin[atomicAdd(&nfin, 1)] = ((uint64_t)lk << 32) | (uint32_t)x;
    }
    for (int sg = w; sg < segs; sg += kTopkThreads / 64) {
      const int lo = off[sg], len = off[sg + 1] - lo;
      for (int p0 = 0; p0 < len; p0 += 64) {
        const int p = p0 + lane;
        const uint64_t x = p < len ? la[lo + p] : 0ull;
        const uint32_t lk = p < len ? key_of_x((uint32_t)(x >> 32)) : 0u;
        if (lk == kth && p < len) {
          const int at = atomicAdd(&ntie, 1);
          if (at < kMaxTie) tg[at] = ((uint64_t)lk << 32) | (uint32_t)x;
        }
        // the list is sorted: past its last entry at or above the k-th logp, stop
        if (__builtin_amdgcn_ballot_w64(p < len && lk >= kth) != ~0ull) break;
      }
    }
    if (tid < segs) {
      const uint32_t bk = seg_bound[base + tid];
      if (bk != 0 && key_of_x(bk) >= kth) atomicOr(&flag, 1);
    }
    __syncthreads();
    exact = flag != 0 || ntie > kMaxTie;
    if (!exact) {
      const int above = nfin, g = ntie, need = k - above;
      for (int i = tid; i < g; i += kTopkThreads) {
        const uint64_t x = tg[i];
        const uint32_t xi = ~(uint32_t)x;                // index
        int rk = 0;
        for (int j = 0; j < g; ++j) rk += (~(uint32_t)tg[j]) < xi ? 1 : 0;
        if (rk < need) fin[above + rk] = x;
      }
      __syncthreads();
      // 3. order by (logp desc, index asc)
      for (int i = tid; i < k; i += kTopkThreads) {
        const uint64_t x = fin[i];
        int pos = 0;
        for (int j = 0; j < k; ++j) pos += fin[j] > x ? 1 : 0;
        const uint32_t ki = (uint32_t)(x >> 32);
        const uint32_t u = (ki & 0x80000000u) ? (ki & 0x7fffffffu) : ~ki;
        row_vals[(int64_t)r * k + pos] = __uint_as_float(u);
        row_idx[(int64_t)r * k + pos] = (int32_t)~(uint32_t)x;
      }
      return;
    }
  }
  // every logit of the row (re-read from memory; rows here are rare)
  const T* row = logits + (int64_t)r * row_stride;
  select_k([&](int i) { return fkey(logp_of<T>(scaled<T>(load_logit(row + i), ts), m, L)); },
           [&](int i) { return i; }, vocab, k, skey, sidx, hist, suf, misc);
  // rank the k chosen by (key desc, idx asc)
  for (int i = tid; i < k; i += kTopkThreads) {
    const uint32_t ki = skey[i];
    const int ii = sidx[i];
    int rank = 0;
    for (int j = 0; j < k; ++j) rank += (skey[j] > ki) || (skey[j] == ki && sidx[j] < ii);
    const uint32_t u = (ki & 0x80000000u) ? (ki & 0x7fffffffu) : ~ki;
    row_vals[(int64_t)r * k + rank] = __uint_as_float(u);
    row_idx[(int64_t)r * k + rank] = ii;
  }
}

// ---------------------------------------------------------------- pass 3
// Per request: the beam best of its pool total = parent[r] + (double)row_vals[r, j]
// by (total desc, pool position r * k + j asc), emitted grouped by row.  Each
// row's list is sorted by logp desc (its totals do not increase along it), so
// an entry's pool rank is its rank in its row plus, in every other row, the
// entries that precede it (a binary search); entries j >= beam of a row
// cannot be selected.
__global__ __launch_bounds__(kTopkThreads) void topk_pool_kernel(int n_rows, int k, int beam, const int32_t* req_row_ptr,
                                                                const double* parent, const float* row_vals,
                                                                const int32_t* row_idx, int32_t* out_parent,
                                                                int32_t* out_token, double* out_score) {
  __shared__ double tot[kMaxPool];
  __shared__ int sel[kMaxPoolRows];
  __shared__ int first[kMaxPoolRows + 1];
  const int tid = threadIdx.x, req = blockIdx.x;
  const int rb = req_row_ptr ? req_row_ptr[req] : 0;
  const int re = req_row_ptr ? req_row_ptr[req + 1] : n_rows;
  int32_t* op = out_parent + (int64_t)req * beam;
  int32_t* ot = out_token + (int64_t)req * beam;
  double* os = out_score + (int64_t)req * beam;
  const bool ok = rb >= 0 && re <= n_rows && rb <= re && (re - rb) <= kMaxPoolRows && (int64_t)(re - rb) * k <= kMaxPool;
  const int nr = ok ? re - rb : 0;
  const int n = nr * k;
  // four entries per thread at a time, their loads issued together
  for (int i0 = 0; i0 < n; i0 += 4 * kTopkThreads) {
    double pv[4];
    float rv[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = min(i0 + u * kTopkThreads + tid, n - 1);
      pv[u] = parent[rb + i / k];
      rv[u] = row_vals[(int64_t)rb * k + i];
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = i0 + u * kTopkThreads + tid;
      if (i < n) tot[i] = pv[u] + (double)rv[u];
    }
  }
  for (int i = tid; i < nr; i += kTopkThreads) sel[i] = 0;
  __syncthreads();
  const int jb = min(k, beam);                      // candidates per row
  int top = 1;
  while (top * 2 <= jb) top *= 2;
  for (int e = tid; e < nr * jb; e += kTopkThreads) {
    const int rr = e / jb, j = e - rr * jb;
    const double t = tot[rr * k + j];
    int rank = j;
    // entries of row o before (rr, j): totals > t, or == t when o < rr -- a
    // prefix of the row, counted over its first jb entries (a count of jb
    // already puts the entry at rank >= beam); sixteen rows' binary searches
    // at a time, with selects rather than branches so that their LDS reads
    // overlap (bitwise & and | keep every read unconditional)
    for (int o0 = 0; o0 < nr && rank < beam; o0 += 16) {
      int pos[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) pos[u] = 0;
      for (int step = top; step > 0; step >>= 1) {
        double y[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          const int o = o0 + u, c = pos[u] + step;
          const bool use = (o < nr) & (o != rr) & (c <= jb);
          y[u] = tot[use ? o * k + c - 1 : 0];
        }
        // the sixteen reads above are issued before any compare waits for one
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          const int o = o0 + u, c = pos[u] + step;
          const bool use = (o < nr) & (o != rr) & (c <= jb);
          pos[u] = (use & ((y[u] > t) | ((y[u] == t) & (o < rr)))) ? c : pos[u];
        }
      }
#pragma unroll
      for (int u = 0; u < 16; ++u) rank += pos[u];
    }
    if (rank < beam) atomicAdd(&sel[rr], 1);
  }
  __syncthreads();
  if (tid == 0) {
    first[0] = 0;
    for (int i = 0; i < nr; ++i) first[i + 1] = first[i] + sel[i];
  }
  __syncthreads();
  for (int e = tid; e < nr * jb; e += kTopkThreads) {
    const int rr = e / jb, j = e - rr * jb;
    if (j < sel[rr]) {
      const int at = first[rr] + j;
      op[at] = rb + rr;
      ot[at] = row_idx[(int64_t)(rb + rr) * k + j];
      os[at] = tot[rr * k + j];
    }
  }
  for (int i = first[nr] + tid; i < beam; i += kTopkThreads) {
    op[i] = -1;
    ot[i] = -1;
    os[i] = -INFINITY;
  }
}

// ---------------------------------------------------------------- two-kernel selection
// The three passes above as two launches for 16-bit logits, with the same
// results:
//  * pass A (topk_units16_kernel): per (row, segment) unit the statistics and
//    the candidates of pass 1, unsorted.  A few workgroups per CU take units
//    in turn and load the next unit while computing the current one (a
//    counter handing out units measured far slower: every workgroup's claims
//    queue on one device-scope atomic).  A wave sums e^x' against
//    0, so that no maximum is needed first and each 16-byte chunk of logits is
//    summed as it lands; only a wave whose largest x' lies outside
//    [-600, 600] sums against that maximum instead, and the unit records it.
//  * pass B (topk_rows16_kernel, one workgroup of sixteen waves per row): the
//    row's log-sum-exp from the unit sums; the k-th largest x' among the
//    candidates by a radix select over their 16-bit keys, run while wave 0
//    takes the logarithm (logp is non-decreasing in x', so the k-th largest
//    logp is the logp of the k-th largest x'); the entries above that logp and
//    its ties of lowest index, ordered by counting; or the exact selection
//    over all logits.  The workgroup that completes a request's last row (an
//    arrival counter per request) then runs pass 3 for the request.
// Row lists go to the pool through agent-scope stores and loads (written
// through to the device's point of coherence).
// Arrival counters (u32 at the start of the workspace, one per request) are
// set to zero by the units pass's first workgroup, so the rows pass of every
// call starts from zero whatever the workspace held (a launch also leaves
// them zero: the last arrival resets its word).
constexpr int kFusedRowCand = 2048;    // segs x cap of one row (two per pass-B thread)
constexpr int kFusedPool = 512;        // rows x min(k, beam) of one request, in LDS
constexpr int kFusedPoolRows = 256;
constexpr int kFusedReqs = 512;
constexpr int kFusedTie = 256;
constexpr int kUnitWgPerCu = 4;        // pass A workgroups per CU
constexpr int kUnitWavesPerSimd = 4;
constexpr int kRowThreads = 1024;      // pass B workgroup
constexpr int kRowWaves = kRowThreads / 64;
constexpr int kRowCandPer = kFusedRowCand / kRowThreads;
constexpr int kPoolSurv = 64;           // pool entries ranked pairwise (16 threads each) after the sample bound
static_assert(kPoolSurv * 16 == kRowThreads, "pairwise pool ranks: 16 threads per entry");
static_assert(kFusedReqs <= kTopkCounterWords, "topk_counter_bytes reserves one counter per request");
static_assert(kFusedRowCand % kRowThreads == 0, "row candidates are spread evenly over the threads");
static_assert(kFusedPool <= kRowThreads, "one pool entry per pass-B thread");

struct FusedTopkArgs {
  const void* logits;
  int64_t row_stride;
  int vocab, seg_len, segs, n_rows, k, cap;
  TempScale ts;
  float* seg_max;
  double* seg_sum;
  int* seg_cnt;
  uint32_t* seg_bound;                 // bits 0..15: boundary key; bit 31: the sum is against seg_max, not 0
  uint64_t* cand;
  uint32_t* ctr;                       // one arrival counter per request
  float* row_vals;
  int32_t* row_idx;
  const double* parent;
  int beam, n_req;
  const int32_t* req_row_ptr;
  int32_t* out_parent;
  int32_t* out_token;
  double* out_score;
};

// Stores written through to the device's coherence point and loads that read
// there (agent scope): another workgroup of the same launch reads them after
// an arrival counter says they are complete.
__device__ __forceinline__ void st_wt(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_wt(int32_t* p, int32_t v) { st_wt(reinterpret_cast<uint32_t*>(p), (uint32_t)v); }
__device__ __forceinline__ void st_wt(float* p, float v) {
  st_wt(reinterpret_cast<uint32_t*>(p), __float_as_uint(v));
}
__device__ __forceinline__ uint32_t ld_co(const uint32_t* p) {
  return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int32_t ld_co(const int32_t* p) { return (int32_t)ld_co(reinterpret_cast<const uint32_t*>(p)); }
__device__ __forceinline__ float ld_co(const float* p) { return __uint_as_float(ld_co(reinterpret_cast<const uint32_t*>(p))); }

// Counts one arrival on ctr and returns the count including it; the word
// returns to zero when the count reaches total.
__device__ __forceinline__ uint32_t arrive(uint32_t* ctr, uint32_t total) {
  const uint32_t n = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
  if (n >= total) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return n;
}

// The 16-bit order key of a 16-bit float pattern.
__device__ __forceinline__ uint32_t key16_of_bits(uint32_t bits16) { return key16x2(bits16) & 0xffffu; }

// The 16-bit float pattern of a 16-bit order key.
__device__ __forceinline__ uint16_t bits_of_key16(uint32_t k16) {
  return (uint16_t)((k16 & 0x8000u) ? (k16 ^ 0x8000u) : (~k16 & 0xffffu));
}

// x' of a 16-bit order key (keys at or below that of -inf give -inf).
template <typename T>
__device__ __forceinline__ float value_of_key16(uint32_t k16) {
  const uint32_t kninf = key16_of_bits(__is_same(T, bf16_t) ? 0xff80u : 0xfc00u);
  return k16 > kninf ? to_f32(__builtin_bit_cast(T, bits_of_key16(k16))) : -INFINITY;
}

// The 16-bit order key of logp(x') (logp is rounded to the logits' format).
template <typename T>
__device__ __forceinline__ uint32_t logp_key16(float xs, float m, float L) {
  return key16_of_bits(bits_of<T>(logp_of<T>(xs, m, L)));
}

// ---------------------------------------------------------------- float64 exp, 256-entry table
// e^d for d in [-708, 708] (callers clamp), Tang's method as exp_neg with a
// 256-entry table: k = rint(d 256 / ln 2), r = d - k ln2/256 (Cody-Waite; the
// high part has 32 significant bits, so k times it is exact for |k| < 2^21),
// e^r - 1 by its degree-4 Taylor polynomial (|r| <= ln2/512: the first omitted
// term, r^5/120, is below 4e-17), times 2^((k mod 256) / 256) from the table
// and 2^floor(k / 256) added to the entry's exponent.
constexpr double kInvLn2x256 = 0x1.71547652b82fep+8;
constexpr double kLn2By256Hi = 0x1.62e42feep-9;
constexpr double kLn2By256Lo = 0x1.a39ef35793c76p-41;

__device__ __forceinline__ void exp_table256_init(double* tab) {
  for (int i = threadIdx.x; i < 256; i += blockDim.x) tab[i] = exp2((double)i / 256.0);
}

__device__ __forceinline__ double exp_t256(double d, const double* tab) {
  const double sh = fma(d, kInvLn2x256, kRoundShift);
  const int k = (int)(uint32_t)(uint64_t)__double_as_longlong(sh);
  const double kf = sh - kRoundShift;
  double r = fma(-kf, kLn2By256Hi, d);
  r = fma(-kf, kLn2By256Lo, r);
  double p = fma(r, 1.0 / 24.0, 1.0 / 6.0);
  p = fma(r, p, 0.5);
  p = fma(r, p, 1.0);
  p *= r;                                           // e^r - 1
  const uint64_t tb = (uint64_t)__double_as_longlong(tab[k & 255]);
  const uint32_t hi = (uint32_t)(tb >> 32) + ((uint32_t)(k >> 8) << 20);
  const double t = __longlong_as_double((long long)(((uint64_t)hi << 32) | (uint32_t)tb));
  return fma(t, p, t);
}

// Two packed 16-bit logits with every negative value below -648 (bf16) or
// -650 (f16) -- and -inf and the negative NaN patterns, past-the-segment
// positions among them -- replaced by that value: one unsigned 16-bit min,
// since negative patterns order by magnitude above 0x8000.
template <typename T>
__device__ __forceinline__ uint32_t clamp_low16(uint32_t u) {
  constexpr unsigned short kLow = __is_same(T, bf16_t) ? 0xc422 : 0xe114;
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_min(__builtin_bit_cast(v2u16, u), (v2u16){kLow, kLow}));
}

template <typename T>
__device__ __forceinline__ float half_value(uint32_t u, int hi) {
  if constexpr (__is_same(T, bf16_t)) return __uint_as_float(hi ? (u & 0xffff0000u) : (u << 16));
  else return (float)__builtin_bit_cast(_Float16, (uint16_t)(hi ? (u >> 16) : (u & 0xffffu)));
}

// acc + the float64 sum of e^x' over words [W0, W1) of a thread's logits,
// against 0.  x' below about -650 (and -inf, and the NaN patterns past the
// segment) count as e^-650: nothing against a sum that an x' of at least -600
// adds e^-600 to (a positive NaN stays NaN, but its key puts the wave on the
// sum against its max).  Four exps at a time, each group's arguments chained
// to the previous group's sum, so that the compiler cannot start every range
// reduction at once (which spills).
template <typename T, int W0, int W1>
__device__ __forceinline__ double exp_sum0(SegVals<T>& x, const double* tab, double acc) {
#pragma unroll
  for (int i = W0; i < W1; i += 2) {
    asm volatile("" : "+v"(acc), "+v"(x.w[i]), "+v"(x.w[i + 1]));
    const uint32_t c[2] = {clamp_low16<T>(x.w[i]), clamp_low16<T>(x.w[i + 1])};
#pragma unroll
    for (int j = 0; j < 4; ++j) acc += exp_t256((double)half_value<T>(c[j >> 1], j & 1), tab);
  }
  return acc;
}

// The float64 sum of e^(x' - mw) over a thread's logits given as 16-bit keys
// (0 when mw is -inf): the sum of a wave whose largest x', mw, lies outside
// [-600, 600].
template <typename T, int NW>
__device__ __forceinline__ double exp_sum_keys(const uint32_t (&kp)[NW], float mw, const double* tab) {
  double acc = 0.0, md = (double)mw;
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    uint32_t u = kp[i];
    asm volatile("" : "+v"(acc), "+v"(u));
    acc += exp_t256(fmax((double)value_of_key16<T>(u & 0xffffu) - md, -700.0), tab);
    acc += exp_t256(fmax((double)value_of_key16<T>(u >> 16) - md, -700.0), tab);
  }
  return mw == -INFINITY ? 0.0 : acc;
}

// Pass A: per (row, segment) unit the statistics and the unsorted candidates
// (pass 1 without its sort).  G workgroups (a few per CU) take their units in
// turn; each issues the next unit's loads as soon as the current unit's
// logits are in registers, so that the float64 exp-sums (VALU-bound) run while the next
// logits stream in.  SCALED: the temperature is not 1 (a separate
// instantiation keeps the common path free of the scaling code).
template <typename T, bool SCALED>
__global__ __launch_bounds__(kTopkThreads, kUnitWavesPerSimd) void topk_units16_kernel(FusedTopkArgs a) {
  __shared__ double tab[256];
  __shared__ float wmax[4];
  __shared__ double wsum[4];
  __shared__ uint32_t wtau[4];
  __shared__ int wslow[4];
  __shared__ int ncand;
  __shared__ uint64_t lc[kMaxCap];
  __shared__ uint4 kst[kPerThread / 8 * kTopkThreads];   // a unit's keys, for the candidate pass
  static_assert(sizeof(T) == 2 && kPerThread == 32, "16 words of two 16-bit logits per thread");
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int segs = a.segs, k = a.k, cap = a.cap, seg_len = a.seg_len, vocab = a.vocab;
  const int units = a.n_rows * segs;
  const int G = gridDim.x;
  const T* logits = reinterpret_cast<const T*>(a.logits);
  constexpr int kWords = kPerThread / 2;
  // the rows pass's arrival counters start every call at zero (it runs after
  // this kernel), whatever the workspace held
  if (blockIdx.x == 0)
    for (int i = tid; i < a.n_req; i += kTopkThreads) st_wt(a.ctr + i, 0u);
  // 16-bit keys of -600 and 600: a wave sums against 0 when its largest x' lies between them
  const uint32_t klo = key16_of_bits(bits_of<T>(-600.0f)), khi = key16_of_bits(bits_of<T>(600.0f));
  // Units go out by columns: with G = 4C workgroups, workgroups col, col + C,
  // col + 2C and col + 3C share the units col, col + C, col + 2C, ..., taking
  // 3 : 2 : 2 : 1 of them in workgroup order.  The dispatcher places one
  // workgroup of each quarter of the grid on every CU, in order, and a CU
  // issues its oldest workgroup first: equal shares left the last quarter
  // finishing far behind the first (measured).  Otherwise every G-th unit.
  const bool quarters = (G & 3) == 0;
  const int C = quarters ? G / 4 : G;
  const int qtr = blockIdx.x / C, col = blockIdx.x - qtr * C;
  const int ncol = (units - col + C - 1) / C;          // units col + i C below units
  constexpr int kShare[5] = {0, 3, 5, 7, 8};           // cumulative eighths of a column
  const int i0 = quarters ? ncol * kShare[qtr] / 8 : 0;
  const int i1 = quarters ? ncol * kShare[qtr + 1] / 8 : ncol;
  SegVals<T> x, xn;
  if (i0 < i1) {
    const int u = col + i0 * C;
    const int r = u / segs, b = (u - r * segs) * seg_len;
    load_raw16<T>(logits + (int64_t)r * a.row_stride + b, min(vocab, b + seg_len) - b, x);
  }
  if (tid == 0) ncand = 0;
  exp_table256_init(tab);
  __syncthreads();                                     // the exp table, ncand
  for (int i = i0; i < i1; ++i) {
    const int u = col + i * C;
    const int un = i + 1 < i1 ? u + C : units;
    const int r = u / segs, s = u - r * segs;
    const int b = s * seg_len;
    // the sum against 0, a 16-byte chunk (4 words) at a time as it lands
    double acc = 0.0;
    if constexpr (SCALED) temp16<T>(a.ts, x, 0, 4);
    acc = exp_sum0<T, 0, 4>(x, tab, acc);
    if constexpr (SCALED) temp16<T>(a.ts, x, 4, 8);
    acc = exp_sum0<T, 4, 8>(x, tab, acc);
    if constexpr (SCALED) temp16<T>(a.ts, x, 8, 12);
    acc = exp_sum0<T, 8, 12>(x, tab, acc);
    // the last chunk has landed (the asm reads it): the next unit's loads
    // (issued with this unit's they would share the memory system and both
    // arrive late together)
    asm volatile("" : "+v"(x.w[12]), "+v"(x.w[13]), "+v"(x.w[14]), "+v"(x.w[15]));
    if (un < units) {
      const int rn = un / segs, bn = (un - rn * segs) * seg_len;
      load_raw16<T>(logits + (int64_t)rn * a.row_stride + bn, min(vocab, bn + seg_len) - bn, xn);
    }
    if constexpr (SCALED) temp16<T>(a.ts, x, 12, 16);
    acc = exp_sum0<T, 12, 16>(x, tab, acc);
    // 16-bit order keys in place of the logits
    v2u16 km2 = {0, 0};
#pragma unroll
    for (int i = 0; i < kWords; ++i) {
      x.w[i] = key16x2(x.w[i]);
      km2 = __builtin_elementwise_max(km2, __builtin_bit_cast(v2u16, x.w[i]));
    }
    const uint32_t kmax = max((uint32_t)km2.x, (uint32_t)km2.y);
    const uint32_t wk = lane63(wave_scan_max(kmax));
    const float mw = value_of_key16<T>(wk);
    const bool slow = wk > khi || wk < klo;              // wave-uniform
    if (slow) acc = exp_sum_keys<T, kWords>(x.w, mw, tab);
    // the wave's kw-th largest per-thread maximum, bit by bit
    const int kw = (k + 3) >> 2;
    uint32_t pref = 0;
    for (int bit = 15; bit >= 0; --bit) {
      const uint32_t c = pref | (1u << bit);
      if (__popcll(__builtin_amdgcn_ballot_w64(kmax >= c)) >= kw) pref = c;
    }
    acc = wave_scan_add_f64(acc);
    if (lane == 63) {
      wmax[w] = mw;
      wsum[w] = acc;
      wtau[w] = pref;
      wslow[w] = slow ? 1 : 0;
    }
    __syncthreads();
    const float m = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    const uint32_t tau = max(1u, min(min(wtau[0], wtau[1]), min(wtau[2], wtau[3])));
    const v2u16 t1 = {(unsigned short)(tau - 1), (unsigned short)(tau - 1)};
    const v2u16 one = {1, 1};
    // one bit per key >= tau: bit i for the low half of word i, bit 16 + i for
    // its high half
    uint32_t cm = 0;
#pragma unroll
    for (int i = 0; i < kWords; ++i)
      cm |= __builtin_bit_cast(uint32_t, __builtin_elementwise_min(
                __builtin_elementwise_sub_sat(__builtin_bit_cast(v2u16, x.w[i]), t1), one)) << i;
    const int mine = __popc(cm);
    const int incl = wave_scan_add(mine);
    int wbase = 0;
    if (lane == 63) wbase = atomicAdd(&ncand, incl);
    int at = (int)lane63((uint32_t)wbase) + incl - mine;
    if (__builtin_amdgcn_ballot_w64(mine > 0)) {
      // the keys go through LDS so that a thread visits only its set bits (a
      // register cannot be indexed per lane); each thread reads back its own
      // words only
#pragma unroll
      for (int c = 0; c < kWords / 4; ++c)
        kst[c * kTopkThreads + tid] = make_uint4(x.w[4 * c], x.w[4 * c + 1], x.w[4 * c + 2], x.w[4 * c + 3]);
      const uint16_t* kh = reinterpret_cast<const uint16_t*>(kst);
      while (cm) {
        const int j = __builtin_ctz(cm), i = j & 15, h = j >> 4;
        cm &= cm - 1;
        const int q = (i >> 2) * kTopkThreads + tid;       // the word's 16-byte chunk
        const uint32_t key = kh[q * 8 + (i & 3) * 2 + h];
        // position (i >> 2) * 256 * 8 + tid * 8 + 2 (i & 3) + h, as seg_pos(2 i + h)
        if (at < cap) lc[at] = ((uint64_t)key << 32) | (uint32_t)~(uint32_t)(b + q * 8 + (i & 3) * 2 + h);
        ++at;
      }
    }
    __syncthreads();
    const int total = ncand;
    const int64_t rs = (int64_t)r * segs + s;
    for (int i = tid; i < min(total, cap); i += kTopkThreads) a.cand[rs * cap + i] = lc[i];
    if (tid == 0) {
      // the waves' sums against one reference: 0, or the unit's max when a wave
      // summed against a max above 600 (or every wave against its own)
      float ref = -INFINITY;
#pragma unroll
      for (int q = 0; q < 4; ++q) ref = fmaxf(ref, wslow[q] ? wmax[q] : 0.0f);
      double sum = 0.0;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float rq = wslow[q] ? wmax[q] : 0.0f;
        if (wsum[q] != 0.0) sum += rq == ref ? wsum[q] : wsum[q] * exp_t256(fmax((double)rq - (double)ref, -700.0), tab);
      }
      a.seg_max[rs] = m;
      a.seg_sum[rs] = sum;
      a.seg_cnt[rs] = total <= cap ? total : -1;
      a.seg_bound[rs] = (tau > 1 ? tau - 1 : 0u) | (ref == 0.0f ? 0u : 0x80000000u);
    }
    __syncthreads();                                   // lc, ncand, wmax.. free again
    if (tid == 0) ncand = 0;
#pragma unroll
    for (int i = 0; i < kWords; ++i) x.w[i] = xn.w[i];
  }
}

// LDS of pass B.
struct RowLds {
  float m, L;
  int exact, nabove, ntie, flag, req, rb, re, bin, rem, lo, shift, nsurv;
  double pt;
  int ppos;
  int off[kMaxSegs + 1];
  uint32_t sbound[kMaxSegs];
  int hist[2][256];
  int req_ptr[kFusedReqs + 1];
  uint64_t fin[kMaxK];
  uint64_t tg[kFusedTie];
  double ptot[kFusedPool];
  int32_t pidx[kFusedPool];
  int sel[kFusedPoolRows];
  int first[kFusedPoolRows + 1];
  int surv[kPoolSurv];
  // the exact selection over all logits
  int xhist[4 * 256];
  int xsuf[257];
  int xmisc[4 + kRowWaves];
  uint32_t skey[kMaxK];
  int32_t sidx[kMaxK];
};

// Inclusive sums within each 16-lane DPP row of a wave (lanes 15, 31, 47 and
// 63 end with their row's total).
__device__ __forceinline__ int row16_scan_add(int x) {
  x += (int)dpp<0x111, 0xf, true>(0, x);
  x += (int)dpp<0x112, 0xf, true>(0, x);
  x += (int)dpp<0x114, 0xf, true>(0, x);
  x += (int)dpp<0x118, 0xf, true>(0, x);
  return x;
}
// Inclusive sums within each 32-lane half of a wave (DPP; lane 31 and lane 63
// end with their half's total).
__device__ __forceinline__ int half_wave_scan_add(int x) {
  x = row16_scan_add(x);
  x += (int)dpp<0x142, 0xa, false>(0, x);
  return x;
}

// One wave: the bin b of hist (256 bins) with suffix(b) >= want > suffix(b + 1),
// suffix(b) counting the entries in bins >= b, and suffix(b + 1) (wave-uniform).
// Lane l holds bins 255 - 4l down to 252 - 4l, so that the inclusive scan over
// lanes is the suffix over bins.  want must not exceed the total.
__device__ __forceinline__ void wave_find_bin(const int* hist, int want, int& bin, int& above) {
  const int lane = threadIdx.x & 63;
  const int b0 = 255 - 4 * lane;
  const int h[4] = {hist[b0], hist[b0 - 1], hist[b0 - 2], hist[b0 - 3]};
  const int incl = wave_scan_add(h[0] + h[1] + h[2] + h[3]);
  int c = incl - (h[0] + h[1] + h[2] + h[3]);          // entries in bins above b0
  int fb = -1, fa = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    if (c < want && c + h[q] >= want) {
      fb = b0 - q;
      fa = c;
    }
    c += h[q];
  }
  const uint64_t hit = __builtin_amdgcn_ballot_w64(fb >= 0);
  const int src = hit ? (int)__builtin_ctzll(hit) : 0;
  bin = __builtin_amdgcn_readlane(fb, src);
  above = __builtin_amdgcn_readlane(fa, src);
}

// Rank by descending key of each of n <= 32 keys in LDS: thread t compares key
// t >> 5 with key t & 31 and the 32 lanes of a key add their comparisons.
// Returns the rank in the lane with (t & 31) == 31 of each key below n, -1
// elsewhere (every thread of the block calls it).
__device__ __forceinline__ int rank32_desc(const uint64_t* v, int n) {
  const int t = threadIdx.x, i = t >> 5, j = t & 31;
  const int c = half_wave_scan_add((i < n && j < n && v[j] > v[i]) ? 1 : 0);
  return (j == 31 && i < n) ? c : -1;
}

// Writes the k entries of fin (composite keys: logp key << 32 | ~index) to row
// r's lists in rank order (every thread of the block calls it).
template <typename T>
__device__ __forceinline__ void store_row(const FusedTopkArgs& a, int r, const uint64_t* fin) {
  const int k = a.k;
  auto put = [&](uint64_t x, int pos) {
    st_wt(a.row_vals + (int64_t)r * k + pos, to_f32(__builtin_bit_cast(T, bits_of_key16((uint32_t)(x >> 32)))));
    st_wt(a.row_idx + (int64_t)r * k + pos, (int32_t)~(uint32_t)x);
  };
  if (k <= 32) {
    const int pos = rank32_desc(fin, k);
    if (pos >= 0) put(fin[threadIdx.x >> 5], pos);
  } else {
    for (int i = threadIdx.x; i < k; i += kRowThreads) {
      const uint64_t x = fin[i];
      int pos = 0;
      for (int j = 0; j < k; ++j) pos += fin[j] > x ? 1 : 0;
      put(x, pos);
    }
  }
}

// The row max mm and S e^-(R - mm) = B, S = sum over the row of e^(x' - mm),
// from the unit statistics held by wave 0 (lane s < segs: unit s's max, sum
// and whether the sum is against that max rather than 0; R the largest
// reference).  Wave 0 only; every lane ends with the same values.
__device__ __forceinline__ void row_sum(bool in, float mu, double su, bool against_max, float& mm, float& R,
                                        double& B) {
  mm = wave_max(mu);
  const float ref = !in ? -INFINITY : against_max ? mu : 0.0f;
  double t = su;
  if (__builtin_amdgcn_ballot_w64(against_max) == 0) {
    R = __builtin_amdgcn_ballot_w64(in) != 0 ? 0.0f : -INFINITY;
  } else {
    R = wave_max(ref);
    t = su != 0.0 ? su * exp((double)ref - (double)R) : 0.0;
  }
  B = __shfl(wave_scan_add_f64(t), 63, 64);
}

// L = fl32(ln S) from row_sum's values.
__device__ __forceinline__ float row_log(float mm, float R, double B) {
  return (float)(log(B) + ((double)R - (double)mm));
}

// Pass 3 for request q (rows [rb, re)) from the row lists written by this
// launch; only each row's first min(k, beam) entries can be chosen (every
// thread of the block; ends with a barrier).  An entry's rank is its position
// in its row plus, in every other row, the entries before it in the order
// (total desc, pool position asc) -- a prefix of that row, found by binary
// search; P adjacent threads share an entry, each taking every P-th row.
__device__ void fused_pool(const FusedTopkArgs& a, int rb, int re, int q, RowLds& sm) {
  const int tid = threadIdx.x, k = a.k, beam = a.beam;
  int32_t* op = a.out_parent + (int64_t)q * beam;
  int32_t* ot = a.out_token + (int64_t)q * beam;
  double* os = a.out_score + (int64_t)q * beam;
  const int nr = re - rb, jb = min(k, beam), n = nr * jb;
  if (tid < n) {
    const int rr = tid / jb, j = tid - rr * jb;
    const float rv = ld_co(a.row_vals + (int64_t)(rb + rr) * k + j);
    const int32_t ri = ld_co(a.row_idx + (int64_t)(rb + rr) * k + j);
    sm.ptot[tid] = a.parent[rb + rr] + (double)rv;
    sm.pidx[tid] = ri;
  }
  for (int i = tid; i < nr; i += kRowThreads) sm.sel[i] = 0;
  __syncthreads();
  // A bound on the beam-th best: the beam-th best (rank beam - 1) of a sample,
  // each row's first ns entries.  Every entry of the top beam is at or before
  // it (beam sampled entries are), so only those -- per row a prefix -- need
  // exact ranks, and their ranks among themselves are their ranks in the pool.
  // (ns a power of two, so that a sample's pool position is a shift and a mask)
  const int ns_max = nr <= kPoolSurv ? min(jb, kPoolSurv / nr) : 0;
  const int lns = ns_max > 0 ? 31 - __builtin_clz(ns_max) : 0;
  const int ns = ns_max > 0 ? 1 << lns : 0;
  const int nsamp = nr * ns;
  auto samp_pos = [&](int i) { return (i >> lns) * jb + (i & (ns - 1)); };
  int S = kPoolSurv + 1;                               // survivors; above kPoolSurv: rank every entry
  if (nsamp >= beam) {
    {
      // sample i = tid >> 4 against samples (tid & 15) + 16 u, summed over the
      // 16 lanes of its DPP row
      const int i = tid >> 4, j0 = tid & 15;
      const int pi = i < nsamp ? samp_pos(i) : 0;
      int c = 0;
      if (i < nsamp) {
        const double ti = sm.ptot[pi];
#pragma unroll
        for (int u = 0; u < kPoolSurv / 16; ++u) {
          const int jj = j0 + 16 * u;
          if (jj < nsamp) {
            const int pj = samp_pos(jj);
            const double tj = sm.ptot[pj];
            c += (tj > ti || (tj == ti && pj < pi)) ? 1 : 0;
          }
        }
      }
      c = row16_scan_add(c);
      if (j0 == 15 && i < nsamp && c == beam - 1) {
        sm.pt = sm.ptot[pi];
        sm.ppos = pi;
      }
    }
    __syncthreads();
    if (tid < 64) {
      // the prefix of row tid at or before the bound, by binary search
      const double pt = sm.pt;
      const int ppos = sm.ppos;
      int c = 0;
      if (tid < nr) {
        int lo = 0, hi = jb;                           // entries [0, lo) qualify, [hi, jb) do not
        while (lo < hi) {
          const int mid = (lo + hi) >> 1, pm = tid * jb + mid;
          const double y = sm.ptot[pm];
          if (y > pt || (y == pt && pm <= ppos)) lo = mid + 1;
          else hi = mid;
        }
        c = lo;
      }
      const int incl = wave_scan_add(c);
      const int tot = __builtin_amdgcn_readlane(incl, 63);
      if (tot <= kPoolSurv)
        for (int j2 = 0; j2 < c; ++j2) sm.surv[incl - c + j2] = tid * jb + j2;
      if (tid == 0) sm.nsurv = tot;
    }
    __syncthreads();
    S = sm.nsurv;
  }
  if (S <= kPoolSurv) {
    // the survivors' ranks: survivor t >> 4 against survivors (t & 15) + 16 u
    const int i = tid >> 4, j0 = tid & 15;
    const int pi = i < S ? sm.surv[i] : 0;
    int c = 0;
    if (i < S) {
      const double ti = sm.ptot[pi];
#pragma unroll
      for (int u = 0; u < kPoolSurv / 16; ++u) {
        const int jj = j0 + 16 * u;
        if (jj < S) {
          const int pj = sm.surv[jj];
          const double tj = sm.ptot[pj];
          c += (tj > ti || (tj == ti && pj < pi)) ? 1 : 0;
        }
      }
    }
    c = row16_scan_add(c);
    if (j0 == 15 && i < S && c < beam) atomicAdd(&sm.sel[pi / jb], 1);
  } else {
    // every entry's rank: P adjacent threads share an entry, each taking every
    // P-th row, and add their counts
    const int P = n <= kRowThreads / 8 ? 8 : n <= kRowThreads / 4 ? 4 : 2;
    const int e = tid / P, part = tid - e * P;
    int cnt = 0;
    int rr = 0, j = 0;
    if (e < n) {
      rr = e / jb;
      j = e - rr * jb;
      const double t = sm.ptot[e];
      int top = 1;
      while (top * 2 <= jb) top *= 2;
      for (int o0 = part; o0 < nr; o0 += 4 * P) {
        int pos[4] = {0, 0, 0, 0};
        for (int step = top; step > 0; step >>= 1) {
          double y[4];
#pragma unroll
          for (int uu = 0; uu < 4; ++uu) {
            const int o = o0 + uu * P, c = pos[uu] + step;
            const bool use = (o < nr) & (o != rr) & (c <= jb);
            y[uu] = sm.ptot[use ? o * jb + c - 1 : 0];
          }
#pragma unroll
          for (int uu = 0; uu < 4; ++uu) {
            const int o = o0 + uu * P, c = pos[uu] + step;
            const bool use = (o < nr) & (o != rr) & (c <= jb);
            pos[uu] = (use & ((y[uu] > t) | ((y[uu] == t) & (o < rr)))) ? c : pos[uu];
          }
        }
        cnt += pos[0] + pos[1] + pos[2] + pos[3];
      }
    }
    for (int sft = 1; sft < P; sft <<= 1) cnt += __shfl_xor(cnt, sft, 64);
    if (e < n && part == 0 && j + cnt < beam) atomicAdd(&sm.sel[rr], 1);
  }
  __syncthreads();
  if (tid < 64) {
    // exclusive prefix of the rows' selection counts, four rows per lane
    int v[4], s4 = 0;
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) {
      const int i = 4 * tid + qq;
      v[qq] = i < nr ? sm.sel[i] : 0;
      s4 += v[qq];
    }
    const int incl = wave_scan_add(s4);
    int base = incl - s4;
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) {
      const int i = 4 * tid + qq;
      if (i < nr) sm.first[i] = base;
      base += v[qq];
    }
    if (tid == 63) sm.first[nr] = incl;
  }
  __syncthreads();
  if (tid < n) {
    const int r2 = tid / jb, j2 = tid - r2 * jb;
    if (j2 < sm.sel[r2]) {
      const int at = sm.first[r2] + j2;
      op[at] = rb + r2;
      ot[at] = sm.pidx[tid];
      os[at] = sm.ptot[tid];
    }
  }
  for (int i = sm.first[nr] + tid; i < beam; i += kRowThreads) {
    op[i] = -1;
    ot[i] = -1;
    os[i] = -INFINITY;
  }
  __syncthreads();
}

// Pass B: per row (one workgroup of sixteen waves each) the selection from
// pass A's output; the workgroup that completes a request's last row (an
// arrival counter per request) runs pass 3 for it.
template <typename T>
__global__ __launch_bounds__(kRowThreads) void topk_rows16_kernel(FusedTopkArgs a) {
  __shared__ RowLds sm;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, r = blockIdx.x;
  const int segs = a.segs, k = a.k, cap = a.cap;
  const int n_req = a.beam > 0 ? a.n_req : 0;
  const int64_t base = (int64_t)r * segs;
  const int lcap = __ffs(cap) - 1;                     // cap is a power of two
  const int nslots = segs << lcap;
  // requests without rows (or with an invalid range) get empty selections
  for (int q = r; q < n_req; q += gridDim.x) {
    const int rb = a.req_row_ptr ? a.req_row_ptr[q] : 0, re = a.req_row_ptr ? a.req_row_ptr[q + 1] : a.n_rows;
    if (!(rb >= 0 && re <= a.n_rows && rb < re))
      for (int i = tid; i < a.beam; i += kRowThreads) {
        a.out_parent[(int64_t)q * a.beam + i] = -1;
        a.out_token[(int64_t)q * a.beam + i] = -1;
        a.out_score[(int64_t)q * a.beam + i] = -INFINITY;
      }
  }
  // one round trip: every candidate slot of the row (slots past a unit's count
  // hold stale words: unused), the unit statistics (wave 0), the request
  // pointers
  uint64_t cv[kRowCandPer];
  const uint64_t* blk = a.cand + base * cap;
#pragma unroll
  for (int q = 0; q < kRowCandPer; ++q) cv[q] = blk[min(q * kRowThreads + tid, nslots - 1)];
  for (int i = tid; i <= n_req; i += kRowThreads)
    sm.req_ptr[i] = a.req_row_ptr ? a.req_row_ptr[i] : (i == 0 ? 0 : a.n_rows);
  float mu = -INFINITY, mm_row = -INFINITY, R_row = 0.0f;
  double su = 0.0, B_row = 0.0;
  bool against_max = false;
  const bool in = lane < segs;
  if (w == 0) {
    const int li = min(lane, segs - 1);
    mu = a.seg_max[base + li];
    su = a.seg_sum[base + li];
    const int c = a.seg_cnt[base + li];
    const uint32_t bd = a.seg_bound[base + li];
    if (!in) {
      mu = -INFINITY;
      su = 0.0;
    }
    against_max = in && (bd >> 31) != 0;
    if (in) sm.sbound[lane] = bd & 0xffffu;
    const int incl = wave_scan_add(in && c > 0 ? c : 0);
    if (in) sm.off[lane + 1] = incl;
    // the radix select's key range: the k-th largest x' key is at least the
    // threshold of any unit holding k candidates (all its candidates reach
    // it), and at most the row max's key
    const uint32_t tau = (bd & 0xffffu) + 1u;
    const uint32_t lo = wave_scan_max(in && c >= k ? tau : 1u);
    const uint32_t hi = wave_scan_max(in ? key16_of_bits(bits_of<T>(mu)) : 0u);
    const uint32_t lo63 = lane63(lo), hi63 = max(lane63(hi), lo63);
    int shift = 0;
    while (((hi63 - lo63) >> shift) >= 256u) ++shift;
    // an overflowed unit, or fewer candidates than k: the exact selection
    const bool over = __builtin_amdgcn_ballot_w64(in && c < 0) != 0 ||
                      __builtin_amdgcn_readlane(incl, segs - 1) < k;
    row_sum(in, mu, su, against_max, mm_row, R_row, B_row);
    if (lane == 0) {
      sm.off[0] = 0;
      sm.exact = over ? 1 : 0;
      sm.nabove = 0;
      sm.ntie = 0;
      sm.req = -1;
      sm.lo = (int)lo63;
      sm.shift = shift;
    }
  }
  if (tid < 256) {
    sm.hist[0][tid] = 0;
    sm.hist[1][tid] = 0;
  }
  __syncthreads();
  // the request holding row r (wave 3): the last q with req_ptr[q] <= r
  if (w == 3 && n_req > 0) {
    int best = -1;
    for (int q = lane; q < n_req; q += 64)
      if (sm.req_ptr[q] <= r) best = q;
    best = (int)wave_scan_max((uint32_t)(best + 1)) - 1;
    if (lane == 63) {
      const int rb = best >= 0 ? sm.req_ptr[best] : 0, re = best >= 0 ? sm.req_ptr[best + 1] : 0;
      const bool ok = best >= 0 && rb >= 0 && re <= a.n_rows && rb <= r && r < re;
      sm.req = ok ? best : -1;
      sm.rb = rb;
      sm.re = re;
    }
  }
  const bool exact0 = sm.exact != 0;
  // the candidates' x' keys (0 for slots past their unit's count)
  uint32_t xk[kRowCandPer];
#pragma unroll
  for (int q = 0; q < kRowCandPer; ++q) {
    const int f = q * kRowThreads + tid, sg = min(f >> lcap, kMaxSegs - 1), p = f & (cap - 1);
    const bool use = f < nslots && p < sm.off[sg + 1] - sm.off[sg];
    xk[q] = use ? (uint32_t)(cv[q] >> 32) & 0xffffu : 0u;
  }
  if (!exact0) {
    // the k-th largest x' key: radix passes over the keys' offsets from lo
    // (one pass when the range spans at most 256 keys), while wave 0 takes
    // the row's log-sum-exp
    const uint32_t lo = (uint32_t)sm.lo;
    const int shift = sm.shift;
#pragma unroll
    for (int q = 0; q < kRowCandPer; ++q)
      if (xk[q] >= lo && xk[q] != 0) atomicAdd(&sm.hist[0][(xk[q] - lo) >> shift], 1);
    __syncthreads();
    if (w == 0 && lane == 0) {
      sm.m = mm_row;
      sm.L = row_log(mm_row, R_row, B_row);
    }
    if (w == 1) {
      int bin, above;
      wave_find_bin(sm.hist[0], k, bin, above);
      if (lane == 0) {
        sm.bin = shift == 0 ? (int)lo + bin : bin;
        sm.rem = k - above;
      }
    }
    __syncthreads();
    if (shift > 0) {
      const uint32_t hb = (uint32_t)sm.bin;
#pragma unroll
      for (int q = 0; q < kRowCandPer; ++q)
        if (xk[q] >= lo && xk[q] != 0 && ((xk[q] - lo) >> shift) == hb)
          atomicAdd(&sm.hist[1][(xk[q] - lo) & ((1u << shift) - 1u)], 1);
      __syncthreads();
      if (w == 1) {
        int bin, above;
        wave_find_bin(sm.hist[1], sm.rem, bin, above);
        if (lane == 0) sm.bin = (int)(lo + (hb << shift) + (uint32_t)bin);
      }
      __syncthreads();
    }
  } else {
    if (w == 0 && lane == 0) {
      sm.m = mm_row;
      sm.L = row_log(mm_row, R_row, B_row);
    }
    __syncthreads();
  }
  const float m = sm.m, L = sm.L;
  bool done = false;
  if (!exact0) {
    // the k-th logp; the entries above it, its tie group, and the units' bounds
    const uint32_t K = logp_key16<T>(value_of_key16<T>((uint32_t)sm.bin), m, L);
#pragma unroll
    for (int q = 0; q < kRowCandPer; ++q) {
      if (xk[q] == 0) continue;
      const uint32_t lk = logp_key16<T>(value_of_key16<T>(xk[q]), m, L);
      const uint64_t e = ((uint64_t)lk << 32) | (uint32_t)cv[q];
      if (lk > K) {
        sm.fin[atomicAdd(&sm.nabove, 1)] = e;
      } else if (lk == K) {
        const int at = atomicAdd(&sm.ntie, 1);
        if (at < kFusedTie) sm.tg[at] = e;
      }
    }
    if (tid < segs) {
      const uint32_t bd = sm.sbound[tid];
      if (bd != 0 && logp_key16<T>(value_of_key16<T>(bd), m, L) >= K) atomicOr(&sm.exact, 1);
    }
    __syncthreads();
    if (!sm.exact && sm.ntie <= kFusedTie) {
      // the need lowest indices of the tie group (largest composite keys)
      const int above = sm.nabove, g = sm.ntie, need = k - above;
      if (g <= 32) {
        const int rk = rank32_desc(sm.tg, g);
        if (rk >= 0 && rk < need) sm.fin[above + rk] = sm.tg[tid >> 5];
      } else {
        for (int i = tid; i < g; i += kRowThreads) {
          const uint64_t x = sm.tg[i];
          int rk = 0;
          for (int jj = 0; jj < g; ++jj) rk += sm.tg[jj] > x ? 1 : 0;
          if (rk < need) sm.fin[above + rk] = x;
        }
      }
      __syncthreads();
      store_row<T>(a, r, sm.fin);
      done = true;
    }
  }
  if (!done) {
    // every logit of the row
    __syncthreads();
    const T* row = reinterpret_cast<const T*>(a.logits) + (int64_t)r * a.row_stride;
    const TempScale ts = a.ts;
    select_k<kRowThreads>([&](int i) { return fkey(logp_of<T>(scaled<T>(load_logit(row + i), ts), m, L)); },
                          [&](int i) { return i; }, a.vocab, k, sm.skey, sm.sidx, sm.xhist, sm.xsuf, sm.xmisc);
    for (int i = tid; i < k; i += kRowThreads) {
      const uint32_t ki = sm.skey[i];
      const int ii = sm.sidx[i];
      int rank = 0;
      for (int jj = 0; jj < k; ++jj) rank += (sm.skey[jj] > ki) || (sm.skey[jj] == ki && sm.sidx[jj] < ii);
      const uint32_t uu = (ki & 0x80000000u) ? (ki & 0x7fffffffu) : ~ki;
      st_wt(a.row_vals + (int64_t)r * k + rank, __uint_as_float(uu));
      st_wt(a.row_idx + (int64_t)r * k + rank, (int32_t)ii);
    }
  }
  if (n_req == 0) return;
  // the row lists are complete before this row's arrival counts
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0) {
    const int q = sm.req;
    sm.flag = q >= 0 && arrive(a.ctr + q, (uint32_t)(sm.re - sm.rb)) == (uint32_t)(sm.re - sm.rb);
  }
  __syncthreads();
  if (sm.flag) fused_pool(a, sm.rb, sm.re, sm.req, sm);
}

// ---------------------------------------------------------------- diverse selection
// Diverse beam search with the Hamming penalty (beam_strategy.py:173-312),
// one workgroup per request over its pool of row top-k choices (row-major:
// choice i = (row rb + i / k, rank i % k)).  Groups pick in turn, each
// max(1, beam / groups) choices not yet taken, by
//   (log_prob - penalty * [token taken by an earlier group]) descending,
// ties to the higher log_prob, then the lower pool position -- the order of the
// reference's two stable sorts (by log_prob over the pool in row order, then by
// the adjusted score; its length normalisation divides every choice of a step
// by the same positive factor and leaves that order unchanged).  The picks are
// emitted grouped by row (rows ascending, each row's children in pick order);
// beyond beam entries the last ones are dropped.
struct DivKey {
  double adj;
  float lp;
  int pos;
};
__device__ __forceinline__ bool div_better(const DivKey& a, const DivKey& b) {
  if (a.pos < 0) return false;
  if (b.pos < 0) return true;
  if (a.adj != b.adj) return a.adj > b.adj;
  if (a.lp != b.lp) return a.lp > b.lp;
  return a.pos < b.pos;
}

__global__ __launch_bounds__(kTopkThreads) void topk_diverse_kernel(int n_rows, int k, int beam, int groups,
                                                                   double penalty, const int32_t* req_row_ptr,
                                                                   const double* parent, const float* row_vals,
                                                                   const int32_t* row_idx, int32_t* out_parent,
                                                                   int32_t* out_token, double* out_score) {
  __shared__ uint8_t state[kMaxPool];        // bit 0: taken; bit 1: token taken by an earlier group
  __shared__ int picks[kMaxK];                // pool positions in pick order
  __shared__ int pick_tok[kMaxK];
  __shared__ DivKey red[kTopkThreads];
  __shared__ int n_picks;
  const int tid = threadIdx.x;
  const int req = blockIdx.x;
  const int rb = req_row_ptr ? req_row_ptr[req] : 0;
  const int re = req_row_ptr ? req_row_ptr[req + 1] : n_rows;
  int32_t* op = out_parent + (int64_t)req * beam;
  int32_t* ot = out_token + (int64_t)req * beam;
  double* os = out_score + (int64_t)req * beam;
  const bool ok = rb >= 0 && re <= n_rows && rb <= re && (int64_t)(re - rb) * k <= kMaxPool;
  const int n = ok ? (re - rb) * k : 0;
  const float* vals = row_vals + (int64_t)rb * k;
  const int32_t* toks = row_idx + (int64_t)rb * k;
  const int per = max(1, beam / groups);
  for (int i = tid; i < n; i += kTopkThreads) state[i] = 0;
  if (tid == 0) n_picks = 0;
  __syncthreads();
  for (int g = 0; g < groups; ++g) {
    const int n0 = n_picks;                   // tokens taken by earlier groups: pick_tok[0, n0)
    for (int i = tid; i < n; i += kTopkThreads) {
      bool hit = false;
      const int t = toks[i];
      for (int j = 0; j < n0; ++j) hit = hit || pick_tok[j] == t;
      state[i] = (uint8_t)((state[i] & 1) | (hit ? 2 : 0));
    }
    __syncthreads();
    for (int s = 0; s < per; ++s) {
      DivKey best{0.0, 0.f, -1};
      for (int i = tid; i < n; i += kTopkThreads) {
        if (state[i] & 1) continue;
        const DivKey c{(double)vals[i] - ((state[i] & 2) ? penalty : 0.0), vals[i], i};
        if (div_better(c, best)) best = c;
      }
      red[tid] = best;
      __syncthreads();
      for (int w = kTopkThreads / 2; w > 0; w >>= 1) {
        if (tid < w && div_better(red[tid + w], red[tid])) red[tid] = red[tid + w];
        __syncthreads();
      }
      const int win = red[0].pos;
      if (win < 0) break;                     // (uniform: every thread reads red[0])
      if (tid == 0) {
        state[win] |= 1;
        picks[n_picks] = win;
        pick_tok[n_picks] = toks[win];
        n_picks += 1;
      }
      __syncthreads();
    }
  }
  __syncthreads();
  const int cnt = n_picks;
  const int keep = min(cnt, beam);
  // emission rank of pick q: picks of lower rows, then earlier picks of its own row
  for (int q = tid; q < cnt; q += kTopkThreads) {
    const int p = picks[q], row = p / k;
    int rank = 0;
    for (int j = 0; j < cnt; ++j) {
      const int rj = picks[j] / k;
      rank += (rj < row) || (rj == row && j < q);
    }
    if (rank < keep) {
      op[rank] = rb + row;
      ot[rank] = toks[p];
      os[rank] = parent[rb + row] + (double)vals[p];
    }
  }
  for (int i = keep + tid; i < beam; i += kTopkThreads) {
    op[i] = -1;
    ot[i] = -1;
    os[i] = -INFINITY;
  }
}

// ---------------------------------------------------------------- static scratch
// Device scratch of be_beam_topk_noalloc: one copy per GPU, alive until the
// process ends.  Host code never passes `topk_scratch` itself to a kernel (on
// the host the name is only a stand-in for the symbol): its device address is
// looked up once per device with hipGetSymbolAddress, with that device
// current, and that address is what the kernels get.  Calls on one GPU share
// the array, so calls that overlap on one GPU (different streams, or host
// threads) race.  The one-launch selection's arrival counters at the start
// of the array start zero (a device array without initialiser is zero-filled
// when the code object loads) and every complete call leaves them zero; every
// other scratch word is written before it is read.
constexpr int64_t kTopkScratchBytes = 8ll << 20;
static __device__ __align__(256) unsigned char topk_scratch[kTopkScratchBytes];

constexpr int kMaxScratchDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_addr[kMaxScratchDevices] = {};

static int topk_scratch_address(hipStream_t st, void** out) {
  int dev = 0;
  if (st != nullptr) {
    hipDevice_t d = 0;
    BE_HIP_CHECK(hipStreamGetDevice(st, &d));
    dev = (int)d;
  } else {
    BE_HIP_CHECK(hipGetDevice(&dev));
  }
  if (dev < 0 || dev >= kMaxScratchDevices)
    return fail(BE_ERR_UNSUPPORTED, "device %d beyond the %d this library tracks", dev, kMaxScratchDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_addr[dev] == nullptr) {
    int cur = 0;
    BE_HIP_CHECK(hipGetDevice(&cur));
    if (cur != dev) BE_HIP_CHECK(hipSetDevice(dev));
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(topk_scratch));
    if (cur != dev) {
      const hipError_t e2 = hipSetDevice(cur);
      if (e2 != hipSuccess) return fail(BE_ERR_HIP, "hipSetDevice(%d) failed: %s", cur, hipGetErrorString(e2));
    }
    if (e != hipSuccess || p == nullptr)
      return fail(BE_ERR_HIP, "hipGetSymbolAddress(topk_scratch) failed on device %d: %s", dev, hipGetErrorString(e));
    g_scratch_addr[dev] = p;
  }
  *out = g_scratch_addr[dev];
  return BE_OK;
}

// Multiprocessor count of the stream's device (cached per device).
static int g_cus[kMaxScratchDevices] = {};

static int topk_device_cus(hipStream_t st, int* out) {
  int dev = 0;
  if (st != nullptr) {
    hipDevice_t d = 0;
    BE_HIP_CHECK(hipStreamGetDevice(st, &d));
    dev = (int)d;
  } else {
    BE_HIP_CHECK(hipGetDevice(&dev));
  }
  if (dev < 0 || dev >= kMaxScratchDevices)
    return fail(BE_ERR_UNSUPPORTED, "device %d beyond the %d this library tracks", dev, kMaxScratchDevices);
  int n = __atomic_load_n(&g_cus[dev], __ATOMIC_RELAXED);
  if (n <= 0) {
    BE_HIP_CHECK(hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev));
    if (n <= 0) n = 1;
    __atomic_store_n(&g_cus[dev], n, __ATOMIC_RELAXED);
  }
  *out = n;
  return BE_OK;
}

}  // namespace be

extern "C" {

int64_t be_beam_topk_workspace_bytes(int n_rows, int vocab, int k) {
  if (n_rows <= 0 || vocab <= 0 || k <= 0) return 0;
  const be::TopkGeom geo = be::topk_geom(n_rows, vocab, k);
  const int64_t ns = (int64_t)n_rows * geo.segs;
  // arrival counters (u32: one per row and per request), seg_sum f64,
  // candidates (u64) x cap, seg_max f32, seg_cnt i32, seg_bound u32
  return be::topk_counter_bytes(n_rows) + ns * 8 + ns * be::topk_cap(k) * 8 + ns * 4 + ns * 4 + ns * 4 + 256;
}

static int topk_launch(const void* logits, int dtype, int n_rows, int vocab, int64_t row_stride, double temperature,
                       int temp_mode, int k,
                 const double* parent_scores, int beam, int n_req, const int32_t* req_row_ptr, int max_req_rows,
                 float* row_vals, int32_t* row_idx, int32_t* out_parent, int32_t* out_token, double* out_score,
                 void* workspace, int64_t workspace_bytes, void* stream) {
  BE_REQUIRE(logits && row_vals && row_idx, "null pointer");
  BE_REQUIRE(dtype == BE_F32 || dtype == BE_F16 || dtype == BE_BF16, "unknown dtype %d", dtype);
  BE_REQUIRE(n_rows > 0 && vocab > 0, "empty logits");
  BE_REQUIRE(k >= 1 && k <= vocab, "k = %d outside [1, vocab = %d]", k, vocab);
  if (k > be::kMaxK) return be::fail(BE_ERR_UNSUPPORTED, "k = %d exceeds %d", k, be::kMaxK);
  BE_REQUIRE(row_stride >= vocab, "row stride %lld < vocab %d", (long long)row_stride, vocab);
  BE_REQUIRE(temperature > 0.0 && isfinite(temperature), "temperature must be positive and finite");
  BE_REQUIRE(temp_mode == BE_TEMP_RECIPROCAL || temp_mode == BE_TEMP_DIVIDE, "unknown temperature mode %d",
             temp_mode);
  // reciprocal: the double reciprocal of the temperature rounded to float, the
  // constant torch multiplies a device tensor by for `logits / temperature`;
  // divide: the float temperature itself
  const float tval = temp_mode == BE_TEMP_DIVIDE ? (float)temperature : (float)(1.0 / temperature);
  const be::TempScale inv_temp{temperature == 1.0 ? 1.0f : tval, temp_mode == BE_TEMP_DIVIDE ? 1 : 0};
  BE_REQUIRE(beam >= 0, "beam must be >= 0");
  if (beam > 0) {
    BE_REQUIRE(parent_scores && out_parent && out_token && out_score, "null selection output");
    BE_REQUIRE(n_req >= 1 && (req_row_ptr != nullptr || n_req == 1), "n_req > 1 needs req_row_ptr");
    BE_REQUIRE(n_req <= 65535, "too many requests");
    if (beam > be::kMaxK) return be::fail(BE_ERR_UNSUPPORTED, "beam = %d exceeds %d", beam, be::kMaxK);
    const int rows = req_row_ptr ? max_req_rows : n_rows;
    BE_REQUIRE(rows >= 0 && rows <= n_rows, "max_req_rows outside [0, n_rows]");
    if ((int64_t)rows * k > be::kMaxPool || rows > be::kMaxPoolRows)
      return be::fail(BE_ERR_UNSUPPORTED, "pool %d x %d exceeds %d entries (or %d rows)", rows, k, be::kMaxPool,
                      be::kMaxPoolRows);
  }
  const int64_t need = be_beam_topk_workspace_bytes(n_rows, vocab, k);
  if (!workspace || workspace_bytes < need)
    return be::fail(BE_ERR_CAPACITY, "top-k workspace needs %lld bytes", (long long)need);
  if (n_rows > 65535) return be::fail(BE_ERR_UNSUPPORTED, "n_rows %d exceeds 65535", n_rows);
  const be::TopkGeom geo = be::topk_geom(n_rows, vocab, k);
  const int cap = be::topk_cap(k);
  if (geo.seg_len > be::kMaxSegLen || geo.segs * cap > be::kMaxRowCand)
    return be::fail(BE_ERR_UNSUPPORTED, "vocab %d with k %d needs segments of %d > %d logits", vocab, k, geo.seg_len,
                    be::kMaxSegLen);
  const int64_t ns = (int64_t)n_rows * geo.segs;
  uint32_t* counters = reinterpret_cast<uint32_t*>(workspace);
  char* ws = reinterpret_cast<char*>(workspace) + be::topk_counter_bytes(n_rows);
  double* seg_sum = reinterpret_cast<double*>(ws);
  uint64_t* cand = reinterpret_cast<uint64_t*>(ws + ns * 8);
  char* tail = ws + ns * 8 + ns * cap * 8;
  float* seg_max = reinterpret_cast<float*>(tail);
  int* seg_cnt = reinterpret_cast<int*>(tail + ns * 4);
  uint32_t* seg_bound = reinterpret_cast<uint32_t*>(tail + ns * 8);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  // two launches for 16-bit logits whose row candidates and request pool fit
  // pass B's registers and LDS arrays
  const int pool_rows = beam > 0 ? (req_row_ptr ? max_req_rows : n_rows) : 0;
  if (dtype != BE_F32 && geo.segs * cap <= be::kFusedRowCand && geo.segs <= be::kMaxSegs &&
      (beam == 0 || (n_req <= be::kFusedReqs && pool_rows <= be::kFusedPoolRows &&
                     (int64_t)pool_rows * std::min(k, beam) <= be::kFusedPool))) {
    be::FusedTopkArgs fa{};
    fa.logits = logits;
    fa.row_stride = row_stride;
    fa.vocab = vocab;
    fa.seg_len = geo.seg_len;
    fa.segs = geo.segs;
    fa.n_rows = n_rows;
    fa.k = k;
    fa.cap = cap;
    fa.ts = inv_temp;
    fa.seg_max = seg_max;
    fa.seg_sum = seg_sum;
    fa.seg_cnt = seg_cnt;
    fa.seg_bound = seg_bound;
    fa.cand = cand;
    fa.ctr = counters;
    fa.row_vals = row_vals;
    fa.row_idx = row_idx;
    fa.parent = parent_scores;
    fa.beam = beam;
    fa.n_req = beam > 0 ? n_req : 0;
    fa.req_row_ptr = req_row_ptr;
    fa.out_parent = out_parent;
    fa.out_token = out_token;
    fa.out_score = out_score;
    int cus = 0;
    const int rc = be::topk_device_cus(st, &cus);
    if (rc != BE_OK) return rc;
    const int g_units = (int)std::min<int64_t>(ns, (int64_t)cus * be::kUnitWgPerCu);
    const bool scaled = inv_temp.t != 1.0f;
    if (dtype == BE_BF16) {
      if (scaled) be::topk_units16_kernel<be::bf16_t, true><<<g_units, be::kTopkThreads, 0, st>>>(fa);
      else be::topk_units16_kernel<be::bf16_t, false><<<g_units, be::kTopkThreads, 0, st>>>(fa);
      be::topk_rows16_kernel<be::bf16_t><<<n_rows, be::kRowThreads, 0, st>>>(fa);
    } else {
      if (scaled) be::topk_units16_kernel<be::f16_t, true><<<g_units, be::kTopkThreads, 0, st>>>(fa);
      else be::topk_units16_kernel<be::f16_t, false><<<g_units, be::kTopkThreads, 0, st>>>(fa);
      be::topk_rows16_kernel<be::f16_t><<<n_rows, be::kRowThreads, 0, st>>>(fa);
    }
    BE_HIP_CHECK(hipGetLastError());
    return BE_OK;
  }
  const dim3 grid(geo.segs, n_rows);
  switch (dtype) {
#define BE_TOPK_CASE(DT, TY, CAND)                                                                                \
  case DT:                                                                                                        \
    be::CAND<TY><<<grid, be::kTopkThreads, 0, st>>>(reinterpret_cast<const TY*>(logits), row_stride, vocab,       \
                                                   geo.seg_len, inv_temp, k, cap, seg_max, seg_sum, seg_cnt,      \
                                                   seg_bound, cand);                                              \
    be::topk_row_kernel<TY><<<n_rows, be::kTopkThreads, 0, st>>>(reinterpret_cast<const TY*>(logits), row_stride,  \
                                                                 vocab, inv_temp, geo.segs, k, cap, seg_max,       \
                                                                 seg_sum, seg_cnt, seg_bound, cand, row_vals,      \
                                                                 row_idx);                                         \
    break;
    BE_TOPK_CASE(BE_F32, float, topk_cand_kernel)
    BE_TOPK_CASE(BE_F16, be::f16_t, topk_cand16_kernel)
    BE_TOPK_CASE(BE_BF16, be::bf16_t, topk_cand16_kernel)
#undef BE_TOPK_CASE
  }
  BE_HIP_CHECK(hipGetLastError());
  if (beam > 0) {
    be::topk_pool_kernel<<<n_req, be::kTopkThreads, 0, st>>>(n_rows, k, beam, req_row_ptr, parent_scores, row_vals,
                                                            row_idx, out_parent, out_token, out_score);
    BE_HIP_CHECK(hipGetLastError());
  }
  return BE_OK;
}

int be_beam_topk(const void* logits, int dtype, int n_rows, int vocab, int64_t row_stride, double temperature,
                 int temp_mode, int k, const double* parent_scores, int beam, int n_req, const int32_t* req_row_ptr,
                 int max_req_rows, float* row_vals, int32_t* row_idx, int32_t* out_parent, int32_t* out_token,
                 double* out_score, void* workspace, int64_t workspace_bytes, void* stream) {
  return topk_launch(logits, dtype, n_rows, vocab, row_stride, temperature, temp_mode, k, parent_scores, beam, n_req,
                     req_row_ptr, max_req_rows, row_vals, row_idx, out_parent, out_token, out_score, workspace,
                     workspace_bytes, stream);
}

int be_beam_topk_noalloc(const void* logits, int dtype, int n_rows, int vocab, int64_t row_stride,
                         double temperature, int temp_mode, int k, const double* parent_scores, int beam, int n_req,
                         const int32_t* req_row_ptr, int max_req_rows, float* row_vals, int32_t* row_idx,
                         int32_t* out_parent, int32_t* out_token, double* out_score, void* stream) {
  const int64_t need = be_beam_topk_workspace_bytes(n_rows, vocab, k);
  if (need > (int64_t)be::kTopkScratchBytes)
    return be::fail(BE_ERR_CAPACITY,
                    "be_beam_topk_noalloc: %d rows x %d logits with k = %d need %lld bytes of scratch, above the "
                    "library's static %lld bytes (use be_beam_topk with a workspace)",
                    n_rows, vocab, k, (long long)need, (long long)be::kTopkScratchBytes);
  void* scratch_dev = nullptr;
  const int rc = be::topk_scratch_address(reinterpret_cast<hipStream_t>(stream), &scratch_dev);
  if (rc != BE_OK) return rc;
  return topk_launch(logits, dtype, n_rows, vocab, row_stride, temperature, temp_mode, k, parent_scores, beam, n_req,
                     req_row_ptr, max_req_rows, row_vals, row_idx, out_parent, out_token, out_score, scratch_dev,
                     (int64_t)be::kTopkScratchBytes, stream);
}

int be_diverse_select(const float* row_vals, const int32_t* row_idx, int n_rows, int k, const double* parent_scores,
                      int n_req, const int32_t* req_row_ptr, int max_req_rows, int beam, int num_groups,
                      double diversity_penalty, int32_t* out_parent, int32_t* out_token, double* out_score,
                      void* stream) {
  BE_REQUIRE(row_vals && row_idx && parent_scores && out_parent && out_token && out_score, "null pointer");
  BE_REQUIRE(n_rows > 0 && k >= 1, "empty pool");
  BE_REQUIRE(beam >= 1 && num_groups >= 1, "beam and num_groups must be positive");
  if (beam > be::kMaxK || num_groups > be::kMaxK)
    return be::fail(BE_ERR_UNSUPPORTED, "beam %d / groups %d exceed %d", beam, num_groups, be::kMaxK);
  BE_REQUIRE(isfinite(diversity_penalty), "diversity penalty must be finite");
  BE_REQUIRE(n_req >= 1 && n_req <= 65535 && (req_row_ptr != nullptr || n_req == 1), "bad request partition");
  const int rows = req_row_ptr ? max_req_rows : n_rows;
  BE_REQUIRE(rows >= 0 && rows <= n_rows, "max_req_rows outside [0, n_rows]");
  if ((int64_t)rows * k > be::kMaxPool)
    return be::fail(BE_ERR_UNSUPPORTED, "pool %d x %d exceeds %d entries", rows, k, be::kMaxPool);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  be::topk_diverse_kernel<<<n_req, be::kTopkThreads, 0, st>>>(n_rows, k, beam, num_groups, diversity_penalty,
                                                             req_row_ptr, parent_scores, row_vals, row_idx,
                                                             out_parent, out_token, out_score);
  BE_HIP_CHECK(hipGetLastError());
  return BE_OK;
}

}  // extern "C"

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
// Pass 1  grid (S, N): per segment max and float64 exp-sum.
// Pass 2  grid (S, N): per segment, exact k best by radix select over the
//         order-preserving uint32 key of logp, ties to the lowest index.
// Pass 3  grid (N):    rank the row's S*k candidates -> sorted row top-k.
// Pass 4  grid (1):    radix select the beam best of the N*k pool (uint64 key
//         of the float64 total, ties to the lowest pool position), emitted in
//         pool-position order = grouped by row, children in selection order.

#include <math.h>

#include <mutex>

#include "common.h"

namespace be {

constexpr int kTopkThreads = 256;
constexpr int kMaxSegLen = 8192;     // keys staged in LDS per segment
constexpr int kMaxSegs = 64;
constexpr int kMaxRowCand = 4096;    // S * k bound for pass 3
constexpr int kMaxPool = 8192;       // N * k bound for pass 4
constexpr int kMaxK = 256;

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
  if (segs * k > kMaxRowCand) segs = kMaxRowCand / k;
  if (segs < 1) segs = 1;
  int seg_len = (vocab + segs - 1) / segs;
  seg_len = (seg_len + 7) & ~7;                           // 16-byte segment starts for 16-bit logits
  segs = (vocab + seg_len - 1) / seg_len;
  return TopkGeom{segs, seg_len};
}

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

// The thread's logits of one segment (n valid positions from seg), scaled by
// the temperature; positions >= n read as `fill`.  16-byte loads when the
// segment start is 16-byte aligned (uniform over the workgroup), else one
// load per logit.
template <typename T>
__device__ __forceinline__ void load_seg(const T* seg, int n, TempScale inv_temp, float fill, float (&x)[kPerThread]) {
  constexpr int V = 16 / (int)sizeof(T);
  if ((reinterpret_cast<uintptr_t>(seg) & 15) == 0) {
#pragma unroll
    for (int c = 0; c < kPerThread / V; ++c) {
      const int p0 = c * (kTopkThreads * V) + (int)threadIdx.x * V;
      if (p0 + V <= n) {
        const uint4 u = *reinterpret_cast<const uint4*>(seg + p0);
        T t[V];
        __builtin_memcpy(t, &u, 16);
#pragma unroll
        for (int e = 0; e < V; ++e) x[c * V + e] = scaled<T>(to_f32(t[e]), inv_temp);
      } else {
#pragma unroll
        for (int e = 0; e < V; ++e) x[c * V + e] = p0 + e < n ? scaled<T>(load_logit(seg + p0 + e), inv_temp) : fill;
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < kPerThread; ++j) {
      const int p = seg_pos<T>(j);
      x[j] = p < n ? scaled<T>(load_logit(seg + p), inv_temp) : fill;
    }
  }
}

__device__ __forceinline__ uint32_t fkey(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ uint64_t dkey(double f) {
  const uint64_t u = (uint64_t)__double_as_longlong(f);
  return (u & 0x8000000000000000ull) ? ~u : (u | 0x8000000000000000ull);
}

__device__ __forceinline__ float block_max(float v, float* red) {
  v = wave_max(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

__device__ __forceinline__ double block_sum_d(double v, double* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

// Block-wide inclusive scans of one int per thread: shuffles inside each wave,
// then the wave totals through LDS (two barriers instead of a barrier pair per
// doubling step).  Suffix: sum over threads >= tid; prefix: threads <= tid.
__device__ __forceinline__ int block_suffix_sum(int v, int* tot /*4*/) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int u = __shfl_down(v, o, 64);
    if (lane + o < 64) v += u;
  }
  if (lane == 0) tot[w] = v;
  __syncthreads();
  for (int x = w + 1; x < 4; ++x) v += tot[x];
  __syncthreads();
  return v;
}
__device__ __forceinline__ int block_prefix_sum(int v, int* tot /*4*/) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int u = __shfl_up(v, o, 64);
    if (lane >= o) v += u;
  }
  if (lane == 63) tot[w] = v;
  __syncthreads();
  for (int x = 0; x < w; ++x) v += tot[x];
  __syncthreads();
  return v;
}

// Exact block-wide selection of the k largest keys, ties broken by the lowest
// position.  keys[0..n) live in LDS.  Writes min(k, n) positions (unordered)
// to out_pos (LDS) and returns that count.  All 256 threads must call it.
template <typename K>
__device__ int block_select(const K* keys, int n, int k, int* out_pos, int* hist /*4*256*/,
                            int* suf /*257*/, int* misc /*8*/) {
  const int tid = threadIdx.x, w = tid >> 6;
  if (n <= k) {
    for (int i = tid; i < n; i += kTopkThreads) out_pos[i] = i;
    __syncthreads();
    return n;
  }
  K prefix = 0, mask = 0;
  int krem = k;
  for (int shift = (int)sizeof(K) * 8 - 8; shift >= 0; shift -= 8) {
    for (int i = tid; i < 4 * 256; i += kTopkThreads) hist[i] = 0;
    __syncthreads();
    for (int i = tid; i < n; i += kTopkThreads) {
      const K key = keys[i];
      if ((key & mask) == prefix) atomicAdd(&hist[w * 256 + (int)((key >> shift) & 255)], 1);
    }
    __syncthreads();
    // suffix sums: suf[d] = #digits >= d
    suf[tid] = block_suffix_sum(hist[tid] + hist[256 + tid] + hist[512 + tid] + hist[768 + tid], misc + 4);
    if (tid == 0) suf[256] = 0;
    __syncthreads();
    if (suf[tid] >= krem && suf[tid + 1] < krem) {   // unique digit
      misc[0] = tid;
      misc[1] = suf[tid + 1];
    }
    __syncthreads();
    const int digit = misc[0];
    krem -= misc[1];
    prefix |= ((K)digit) << shift;
    mask |= ((K)255) << shift;
    __syncthreads();
  }
  // keys > prefix: exactly k - krem of them; keys == prefix: the krem lowest positions
  if (tid == 0) misc[2] = 0;
  __syncthreads();
  const int per = (n + kTopkThreads - 1) / kTopkThreads;
  const int b = tid * per, e = min(n, b + per);
  int eq = 0;
  for (int i = b; i < e; ++i) {
    const K key = keys[i];
    if (key > prefix) out_pos[atomicAdd(&misc[2], 1)] = i;
    else if (key == prefix) ++eq;
  }
  // exclusive scan of eq over threads (in position order)
  int rank = block_prefix_sum(eq, misc + 4) - eq;
  const int ngt = k - krem;
  for (int i = b; i < e && rank < krem; ++i)
    if (keys[i] == prefix) out_pos[ngt + rank++] = i;
  __syncthreads();
  return k;
}

// block_select over keys held in registers by the segment kernel: the
// thread's key j sits at segment position seg_pos<T>(j), present when that
// position is < n.  Exact k largest, ties to the lowest position; writes
// min(k, n) positions (unordered) to out_pos and their keys to out_key and
// returns that count.  All 256 threads must call it.
template <typename T>
__device__ int block_select_regs(const uint32_t (&kr)[kPerThread], int n, int k, int* out_pos, uint32_t* out_key,
                                 int* hist /*4*256*/, int* suf /*257*/, int* misc /*8*/) {
  constexpr int V = 16 / (int)sizeof(T);
  const int tid = threadIdx.x, w = tid >> 6;
  if (n <= k) {
#pragma unroll
    for (int j = 0; j < kPerThread; ++j) {
      const int p = seg_pos<T>(j);
      if (p < n) {
        out_pos[p] = p;
        out_key[p] = kr[j];
      }
    }
    __syncthreads();
    return n;
  }
  uint32_t prefix = 0, mask = 0;
  int krem = k;
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int i = tid; i < 4 * 256; i += kTopkThreads) hist[i] = 0;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kPerThread; ++j)
      if (seg_pos<T>(j) < n && (kr[j] & mask) == prefix) atomicAdd(&hist[w * 256 + (int)((kr[j] >> shift) & 255u)], 1);
    __syncthreads();
    suf[tid] = block_suffix_sum(hist[tid] + hist[256 + tid] + hist[512 + tid] + hist[768 + tid], misc + 4);
    if (tid == 0) suf[256] = 0;
    __syncthreads();
    if (suf[tid] >= krem && suf[tid + 1] < krem) {   // unique digit
      misc[0] = tid;
      misc[1] = suf[tid + 1];
    }
    __syncthreads();
    krem -= misc[1];
    prefix |= ((uint32_t)misc[0]) << shift;
    mask |= 255u << shift;
    __syncthreads();
  }
  // keys > prefix: exactly k - krem of them; keys == prefix: the krem lowest
  // positions, ranked chunk by chunk (chunk c of every thread precedes chunk
  // c + 1 in position order; inside a chunk, threads in order)
  if (tid == 0) misc[2] = 0;
  __syncthreads();
  const int ngt = k - krem;
  int base = 0;
#pragma unroll
  for (int c = 0; c < kPerThread / V; ++c) {
    int eq = 0;
#pragma unroll
    for (int e = 0; e < V; ++e) {
      const int j = c * V + e;
      if (seg_pos<T>(j) < n) {
        if (kr[j] > prefix) {
          const int at = atomicAdd(&misc[2], 1);
          out_pos[at] = seg_pos<T>(j);
          out_key[at] = kr[j];
        } else if (kr[j] == prefix) {
          ++eq;
        }
      }
    }
    const int incl = block_prefix_sum(eq, misc + 4);
    const int chunk_total = misc[4] + misc[5] + misc[6] + misc[7];
    int rank = base + incl - eq;
#pragma unroll
    for (int e = 0; e < V; ++e) {
      const int j = c * V + e;
      if (seg_pos<T>(j) < n && kr[j] == prefix) {
        if (rank < krem) {
          out_pos[ngt + rank] = seg_pos<T>(j);
          out_key[ngt + rank] = prefix;
        }
        ++rank;
      }
    }
    base += chunk_total;
    __syncthreads();   // the wave totals are rewritten by the next chunk's scan
  }
  __syncthreads();
  return k;
}

// ---------------------------------------------------------------- pass 1
template <typename T>
__global__ __launch_bounds__(kTopkThreads) void topk_stats_kernel(const T* logits, int64_t row_stride, int vocab,
                                                                 int seg_len, TempScale inv_temp, float* seg_max,
                                                                 double* seg_sum) {
  __shared__ float redf[4];
  __shared__ double redd[4];
  const int s = blockIdx.x, r = blockIdx.y, segs = gridDim.x;
  constexpr int kPer = kPerThread;                   // logits per thread, read once
  const T* row = logits + (int64_t)r * row_stride;
  const int b = s * seg_len, n = min(vocab, b + seg_len) - b;
  float x[kPer];
  load_seg<T>(row + b, n, inv_temp, -INFINITY, x);
  // each thread sums against its own maximum (no wait for the block's), then
  // rescales by exp(m_t - m); a thread whose logits are all -inf adds 0
  float mt = -INFINITY;
#pragma unroll
  for (int j = 0; j < kPer; ++j) mt = fmaxf(mt, x[j]);
  double acc = 0.0;
  if (mt != -INFINITY) {
    const double md = (double)mt;
#pragma unroll
    for (int j = 0; j < kPer; ++j)
      if (seg_pos<T>(j) < n) acc += exp((double)x[j] - md);
  }
  const float m = block_max(mt, redf);
  if (mt != -INFINITY) acc *= exp((double)mt - (double)m);
  acc = block_sum_d(acc, redd);
  if (threadIdx.x == 0) {
    seg_max[(int64_t)r * segs + s] = m;
    seg_sum[(int64_t)r * segs + s] = acc;
  }
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

// ---------------------------------------------------------------- pass 2
// Block-wide bitonic sort, descending, of one value per thread (256 values):
// partners closer than 64 lanes exchange by shuffle, farther ones through LDS.
template <typename K>
__device__ K block_sort_desc(K v, K* xch) {
  const int tid = threadIdx.x;
#pragma unroll 1
  for (int size = 2; size <= kTopkThreads; size <<= 1) {
#pragma unroll 1
    for (int j = size >> 1; j > 0; j >>= 1) {
      K p;
      if (j >= 64) {
        xch[tid] = v;
        __syncthreads();
        p = xch[tid ^ j];
        __syncthreads();
      } else if constexpr (sizeof(K) == 8) {
        const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)v, j, 64);
        const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), j, 64);
        p = ((K)hi << 32) | lo;
      } else {
        p = (K)__shfl_xor((int)v, j, 64);
      }
      const bool lower = (tid & j) == 0, first_half = (tid & size) == 0;
      // descending blocks where first_half: the lower index keeps the larger value
      v = (lower == first_half) ? (v > p ? v : p) : (v < p ? v : p);
    }
  }
  return v;
}

// Wave-wide bitonic sort, descending, of one value per lane (64 values).
template <typename K>
__device__ K wave_sort_desc(K v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int size = 2; size <= 64; size <<= 1) {
#pragma unroll
    for (int j = size >> 1; j > 0; j >>= 1) {
      K p;
      if constexpr (sizeof(K) == 8) {
        const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)v, j, 64);
        const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), j, 64);
        p = ((K)hi << 32) | lo;
      } else {
        p = (K)__shfl_xor((int)v, j, 64);
      }
      const bool lower = (lane & j) == 0, first_half = (lane & size) == 0;
      v = (lower == first_half) ? (v > p ? v : p) : (v < p ? v : p);
    }
  }
  return v;
}

// Per segment the exact k best logp (ties to the lowest index), emitted in
// ascending index order.  Each wave sorts its 64 per-thread maxima; the
// ceil(k/4)-th largest of every wave are, with the larger ones above them,
// at least k distinct elements, so the smallest of the four is a lower bound
// of the segment's k-th largest key.  The elements at or above it are
// collected as (key, position) composites; up to 64 of them are sorted by one
// wave, up to 256 by the workgroup, more fall back to the radix select over
// all keys.
template <typename T>
__global__ __launch_bounds__(kTopkThreads) void topk_segment_kernel(const T* logits, int64_t row_stride, int vocab,
                                                                   int seg_len, TempScale inv_temp, int k,
                                                                   const float* seg_max, const double* seg_sum,
                                                                   float* cand_val, int32_t* cand_idx) {
  constexpr int kPer = kPerThread;                   // keys per thread (kept in registers)
  __shared__ int pos[kMaxK];
  __shared__ uint32_t selkey[kMaxK];
  __shared__ int hist[4 * 256];
  __shared__ int suf[257];
  __shared__ int misc[8];
  __shared__ uint64_t comp[kTopkThreads];
  __shared__ uint32_t wtau[4];
  __shared__ double terms[64];
  __shared__ float mL[2];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int s = blockIdx.x, r = blockIdx.y, segs = gridDim.x;
  const T* row = logits + (int64_t)r * row_stride;
  const int b = s * seg_len, e = min(vocab, b + seg_len), n = e - b;
  // this thread's logits (positions seg_pos(j)), loaded before the row
  // normaliser so that the two latencies overlap
  float xs[kPer];
  load_seg<T>(row + b, n, inv_temp, 0.f, xs);
  float m, L;
  if (tid == 0) misc[3] = 0;                         // candidate count
  row_norm_block(seg_max, seg_sum, r, segs, m, L, terms, mL);
  // keys (real keys are > 0)
  uint32_t kr[kPer];
  uint32_t kmax = 0;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int i = seg_pos<T>(j);
    uint32_t key = 0;
    if (i < n) key = fkey(logp_of<T>(xs[j], m, L));
    kr[j] = key;
    kmax = key > kmax ? key : kmax;
  }
  const int kw = (k + 3) >> 2;                       // <= 64
  const uint32_t ws = wave_sort_desc<uint32_t>(kmax);
  if (lane == kw - 1) wtau[w] = ws;
  __syncthreads();
  const uint32_t t0 = min(min(wtau[0], wtau[1]), min(wtau[2], wtau[3]));
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int i = seg_pos<T>(j);
    if (i < n && kr[j] >= t0) {
      const int at = atomicAdd(&misc[3], 1);
      if (at < kTopkThreads) comp[at] = ((uint64_t)kr[j] << 32) | (uint32_t)(0xffffffffu - (uint32_t)i);
    }
  }
  __syncthreads();
  const int total = misc[3];
  int cnt = k;
  if (n <= k || total > kTopkThreads) {
    cnt = block_select_regs<T>(kr, n, k, pos, selkey, hist, suf, misc);
  } else if (total <= 64) {
    if (w == 0) {
      const uint64_t v = wave_sort_desc<uint64_t>(lane < total ? comp[lane] : 0ull);
      if (lane < k) {
        pos[lane] = (int)(0xffffffffu - (uint32_t)v);
        selkey[lane] = (uint32_t)(v >> 32);
      }
    }
    __syncthreads();
  } else {
    const uint64_t v = tid < total ? comp[tid] : 0ull;
    __syncthreads();
    const uint64_t sorted = block_sort_desc<uint64_t>(v, comp);
    if (tid < k) {
      pos[tid] = (int)(0xffffffffu - (uint32_t)sorted);
      selkey[tid] = (uint32_t)(sorted >> 32);
    }
    __syncthreads();
  }
  float* cv = cand_val + ((int64_t)r * segs + s) * k;
  int32_t* ci = cand_idx + ((int64_t)r * segs + s) * k;
  // emit in ascending vocabulary index, so that candidate order = index order
  for (int j = tid; j < cnt; j += kTopkThreads) {
    const int p = pos[j];
    int rank = 0;
    for (int t = 0; t < cnt; ++t) rank += (pos[t] < p);
    const uint32_t key = selkey[j];
    const uint32_t u = (key & 0x80000000u) ? (key & 0x7fffffffu) : ~key;
    cv[rank] = __uint_as_float(u);
    ci[rank] = b + p;
  }
  for (int j = cnt + tid; j < k; j += kTopkThreads) {
    cv[j] = -INFINITY;
    ci[j] = -1;   // empty slot (segment shorter than k)
  }
}

// ---------------------------------------------------------------- pass 3
// Candidates are segment-major and index-ascending inside a segment, so their
// position order is vocabulary order: the radix select's lowest-position tie
// rule is the lowest-index rule.  The k selected are then ranked among
// themselves by (value desc, index asc).
__global__ __launch_bounds__(kTopkThreads) void topk_row_kernel(int segs, int k, const float* cand_val,
                                                               const int32_t* cand_idx, float* row_vals,
                                                               int32_t* row_idx) {
  __shared__ uint32_t keys[kMaxRowCand];
  __shared__ int pos[kMaxK];
  __shared__ int hist[4 * 256];
  __shared__ int suf[257];
  __shared__ int misc[8];
  const int r = blockIdx.x;
  const int c = segs * k;
  const float* cv = cand_val + (int64_t)r * c;
  const int32_t* ci = cand_idx + (int64_t)r * c;
  for (int i = threadIdx.x; i < c; i += kTopkThreads) keys[i] = (ci[i] < 0) ? 0u : fkey(cv[i]);
  __syncthreads();
  const int cnt = block_select<uint32_t>(keys, c, k, pos, hist, suf, misc);
  for (int i = threadIdx.x; i < cnt; i += kTopkThreads) {
    const int p = pos[i];
    const uint32_t kp = keys[p];
    int rank = 0;
    for (int j = 0; j < cnt; ++j) {
      const uint32_t kj = keys[pos[j]];
      rank += (kj > kp) || (kj == kp && pos[j] < p);
    }
    row_vals[(int64_t)r * k + rank] = cv[p];
    row_idx[(int64_t)r * k + rank] = ci[p];
  }
}

// ---------------------------------------------------------------- pass 4
// grid.x = request; its rows are [req_row_ptr[r], req_row_ptr[r+1]) (all rows
// when req_row_ptr is null).  Parents are emitted as global row indices.
__global__ __launch_bounds__(kTopkThreads) void topk_global_kernel(int n_rows, int k, int beam,
                                                                  const int32_t* req_row_ptr, const double* parent,
                                                                  const float* row_vals, const int32_t* row_idx,
                                                                  int32_t* out_parent, int32_t* out_token,
                                                                  double* out_score) {
  __shared__ uint64_t keys[kMaxPool];
  __shared__ int pos[kMaxK];
  __shared__ int hist[4 * 256];
  __shared__ int suf[257];
  __shared__ int misc[8];
  const int req = blockIdx.x;
  const int rb = req_row_ptr ? req_row_ptr[req] : 0;
  const int re = req_row_ptr ? req_row_ptr[req + 1] : n_rows;
  int32_t* op = out_parent + (int64_t)req * beam;
  int32_t* ot = out_token + (int64_t)req * beam;
  double* os = out_score + (int64_t)req * beam;
  const bool ok = rb >= 0 && re <= n_rows && rb <= re && (int64_t)(re - rb) * k <= kMaxPool;
  const int n = ok ? (re - rb) * k : 0;
  for (int i = threadIdx.x; i < n; i += kTopkThreads) {
    const int r = rb + i / k;
    keys[i] = dkey(parent[r] + (double)row_vals[(int64_t)rb * k + i]);
  }
  __syncthreads();
  const int cnt = block_select<uint64_t>(keys, n, beam, pos, hist, suf, misc);
  // emit in pool-position order: rows ascending, children in selection order
  for (int i = threadIdx.x; i < cnt; i += kTopkThreads) {
    const int p = pos[i];
    int rank = 0;
    for (int j = 0; j < cnt; ++j) rank += (pos[j] < p);
    const int r = rb + p / k;
    op[rank] = r;
    ot[rank] = row_idx[(int64_t)rb * k + p];
    os[rank] = parent[r] + (double)row_vals[(int64_t)rb * k + p];
  }
  for (int i = cnt + threadIdx.x; i < beam; i += kTopkThreads) {
    op[i] = -1;
    ot[i] = -1;
    os[i] = -INFINITY;
  }
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
// threads) race.  Every kernel writes the scratch words it reads before it
// reads them, so nothing has to be cleared between calls.
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

}  // namespace be

extern "C" {

int64_t be_beam_topk_workspace_bytes(int n_rows, int vocab, int k) {
  if (n_rows <= 0 || vocab <= 0 || k <= 0) return 0;
  const be::TopkGeom geo = be::topk_geom(n_rows, vocab, k);
  const int64_t ns = (int64_t)n_rows * geo.segs;
  return ns * 4 + ns * 8 + ns * k * 4 + ns * k * 4 + 256;
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
    if ((int64_t)rows * k > be::kMaxPool)
      return be::fail(BE_ERR_UNSUPPORTED, "pool %d x %d exceeds %d entries", rows, k, be::kMaxPool);
  }
  const int64_t need = be_beam_topk_workspace_bytes(n_rows, vocab, k);
  if (!workspace || workspace_bytes < need)
    return be::fail(BE_ERR_CAPACITY, "top-k workspace needs %lld bytes", (long long)need);
  if (n_rows > 65535) return be::fail(BE_ERR_UNSUPPORTED, "n_rows %d exceeds 65535", n_rows);
  const be::TopkGeom geo = be::topk_geom(n_rows, vocab, k);
  if (geo.seg_len > be::kMaxSegLen || geo.segs * k > be::kMaxRowCand)
    return be::fail(BE_ERR_UNSUPPORTED, "vocab %d with k %d needs segments of %d > %d logits", vocab, k, geo.seg_len,
                    be::kMaxSegLen);
  const int64_t ns = (int64_t)n_rows * geo.segs;
  char* ws = reinterpret_cast<char*>(workspace);
  double* seg_sum = reinterpret_cast<double*>(ws);
  float* seg_max = reinterpret_cast<float*>(ws + ns * 8);
  float* cand_val = reinterpret_cast<float*>(ws + ns * 12);
  int32_t* cand_idx = reinterpret_cast<int32_t*>(ws + ns * 12 + ns * k * 4);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid(geo.segs, n_rows);
  switch (dtype) {
#define BE_TOPK_CASE(DT, TY)                                                                                   \
  case DT:                                                                                                     \
    be::topk_stats_kernel<TY><<<grid, be::kTopkThreads, 0, st>>>(reinterpret_cast<const TY*>(logits), row_stride, \
                                                                 vocab, geo.seg_len, inv_temp, seg_max, seg_sum); \
    be::topk_segment_kernel<TY><<<grid, be::kTopkThreads, 0, st>>>(reinterpret_cast<const TY*>(logits),        \
                                                                   row_stride, vocab, geo.seg_len, inv_temp, k,   \
                                                                   seg_max, seg_sum, cand_val, cand_idx);       \
    break;
    BE_TOPK_CASE(BE_F32, float)
    BE_TOPK_CASE(BE_F16, be::f16_t)
    BE_TOPK_CASE(BE_BF16, be::bf16_t)
#undef BE_TOPK_CASE
  }
  BE_HIP_CHECK(hipGetLastError());
  be::topk_row_kernel<<<n_rows, be::kTopkThreads, 0, st>>>(geo.segs, k, cand_val, cand_idx, row_vals, row_idx);
  BE_HIP_CHECK(hipGetLastError());
  if (beam > 0) {
    be::topk_global_kernel<<<n_req, be::kTopkThreads, 0, st>>>(n_rows, k, beam, req_row_ptr, parent_scores,
                                                              row_vals, row_idx, out_parent, out_token, out_score);
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

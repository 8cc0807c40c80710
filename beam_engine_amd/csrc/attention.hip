// Paged decode attention for flat / cascade / tree work lists on gfx950.
//
// One work-list format serves every strategy.  A work item is a tile of
// queries (a contiguous slice of q_index) attending to a contiguous token range
// of one paged group (a slice of the plan's page list).  The attention kernel
// runs one workgroup per (item, KV head) and writes either the final output
// (a query with a single item) or a partial (o, lse) row that the merge kernel
// combines by log-sum-exp.  The reference computes the same quantities with
// FlashInfer's MultiLevelCascadeAttentionWrapper (models/modeling_llama.py:
// 321-367, 732-755) and the FastTree Triton kernels
// (attention/fasttree/kernel.py:5-285).

#include <math.h>
#include <stdarg.h>

#include <algorithm>
#include <vector>

#include "attention.h"

namespace be {

// ------------------------------------------------------------------ plan layout
// Device plan = int32 words:
//   items      [num_items][8]   WorkItem
//   q_index    [num_queries]     query ids referenced by items
//   pages      [sum of level page lists]
//   merge_q    [num_merge]       queries the merge kernel combines
//   merge_ptr  [num_merge + 1]   CSR into merge_rows
//   merge_rows [...]             partial rows of each merged query
struct WorkItem {
  int32_t q_begin;     // first entry of q_index
  int32_t q_count;     // queries in the tile
  int32_t page_begin;  // first entry of pages[] of the item's group
  int32_t tok_begin;   // first group token covered (a multiple of 32)
  int32_t tok_count;   // tokens covered, > 0
  int32_t out_row;     // first partial row, or -1: write the final output
  int32_t vis0;        // causal: group tokens its first query sees, unclamped (query j: vis0 + j); else kNoCausal
  int32_t pad1;
};
constexpr int32_t kNoCausal = 0x3fffffff;
static_assert(sizeof(WorkItem) == 32, "WorkItem is 8 int32 words");

constexpr int kMaxRows = 32;       // rows (queries x GQA group) per VALU workgroup
constexpr int kMaxTileRows = 128;  // rows per MFMA workgroup (8 row tiles of 16)

struct AttnArgs {
  const void* q;
  int64_t q_sn, q_sh;
  const void* kv;
  void* out;
  int64_t o_sn, o_sh;
  float* out_lse;
  float* part_o;      // [rows, Hq, D]
  float* part_lse;    // [rows, Hq]
  const WorkItem* items;
  const int32_t* q_index;
  const int32_t* pages;
  // fused merge (null counters: the separate merge kernel runs instead)
  const int32_t* q_merge;      // per query: merge-list index or -1
  const int32_t* merge_ptr;    // CSR of partial rows per merge-list entry
  const int32_t* merge_rows;
  int32_t* counters;           // [num_merge][hkv] arrivals, zero between runs
  const int32_t* live_items;   // fixed layout: live item count (surplus workgroups exit)
  int page_size, hkv, hq, g;
  float scale_log2;   // sm_scale * log2(e)
};

struct MergeArgs {
  const float* part_o;
  const float* part_lse;
  const int32_t* merge_q;
  const int32_t* merge_ptr;
  const int32_t* merge_rows;
  void* out;
  int64_t o_sn, o_sh;
  float* out_lse;
  const int32_t* live;         // fixed layout: live entry count (surplus workgroups exit)
  int hq;
};

// Element offset of (page, kv, slot, head, 0) in a [P, 2, page, Hkv, D] layer.
__device__ __forceinline__ int64_t kv_off(int page, int kvsel, int slot, int head, int page_size,
                                          int hkv, int d) {
  return ((((int64_t)page * 2 + kvsel) * page_size + slot) * hkv + head) * (int64_t)d;
}

// Writes the finished state of one row: o = acc / l, lse = (m + log2 l) ln 2.
template <typename T>
__device__ __forceinline__ void store_row_lse(const AttnArgs& a, const WorkItem& it, int j, int head,
                                              float m2, float l) {
  float lse = (l > 0.f) ? (m2 + log2f(l)) * 0.69314718055994531f : -INFINITY;
  if (it.out_row < 0) {
    if (a.out_lse) {
      int qi = a.q_index[it.q_begin + j];
      a.out_lse[(int64_t)qi * a.hq + head] = lse;
    }
  } else {
    a.part_lse[(int64_t)(it.out_row + j) * a.hq + head] = lse;
  }
}

// Fused split-K merge.  Called by every thread of a workgroup after it wrote
// its partial rows.  For each query of the item the workgroup counts its
// arrival on (query, kv head); the workgroup that completes the count merges
// the g heads of that query from every partial row by log-sum-exp, writes the
// output and resets the counter for the next run.  The release fence makes
// this workgroup's partial rows visible device-wide (all XCD L2s) before its
// arrival is counted; the acquire fence orders the merger's reads after it.
template <typename T, int D>
__device__ void fused_merge_epilogue(const AttnArgs& a, const WorkItem& it, int kvh, int* s_last) {
  __threadfence();
  __syncthreads();
  const int tid = threadIdx.x;
  if (tid < it.q_count) {
    const int qi = a.q_index[it.q_begin + tid];
    const int mi = a.q_merge[qi];
    const int expect = a.merge_ptr[mi + 1] - a.merge_ptr[mi];
    const int old = __hip_atomic_fetch_add(&a.counters[(int64_t)mi * a.hkv + kvh], 1, __ATOMIC_ACQ_REL,
                                           __HIP_MEMORY_SCOPE_AGENT);
    s_last[tid] = (old == expect - 1) ? mi : -1;
  }
  __syncthreads();
  bool fenced = false;
  for (int j = 0; j < it.q_count; ++j) {
    const int mi = s_last[j];
    if (mi < 0) continue;
    if (!fenced) {
      __threadfence();
      fenced = true;
    }
    const int qi = a.q_index[it.q_begin + j];
    const int rb = a.merge_ptr[mi], re = a.merge_ptr[mi + 1];
    // thread -> (head hh, column d); g * D elements over 256 threads
    for (int e = tid; e < a.g * D; e += 256) {
      const int hh = e / D, d = e - hh * D, head = kvh * a.g + hh;
      float M = -INFINITY;
      for (int r = rb; r < re; ++r) M = fmaxf(M, a.part_lse[(int64_t)a.merge_rows[r] * a.hq + head]);
      float z = 0.f, acc = 0.f;
      if (M != -INFINITY) {
        for (int r = rb; r < re; ++r) {
          const int64_t row = (int64_t)a.merge_rows[r] * a.hq + head;
          const float wgt = expf(a.part_lse[row] - M);
          z += wgt;
          acc += wgt * a.part_o[row * D + d];
        }
      }
      T* op = reinterpret_cast<T*>(a.out) + (int64_t)qi * a.o_sn + (int64_t)head * a.o_sh;
      op[d] = from_f32<T>(z > 0.f ? acc / z : 0.f);
      if (d == 0 && a.out_lse) a.out_lse[(int64_t)qi * a.hq + head] = (z > 0.f) ? M + logf(z) : -INFINITY;
    }
    if (tid == 0) a.counters[(int64_t)mi * a.hkv + kvh] = 0;
  }
}

// ================================================================== MFMA kernel
// bf16/fp16 storage, D in {64, 128, 256}, up to 16*RT rows (queries x GQA
// group) per workgroup.
//
// The workgroup streams its token range in 64-token tiles through LDS: all
// 256 threads load a tile with 16-byte loads (16 consecutive lanes read one
// 256-byte K or V row of a page), the next tile's loads are issued before the
// current tile is computed (register prefetch), and the page ids of the item
// are staged in LDS once.  K is kept row-major with its 16-byte chunks
// XOR-swizzled by token; V is stored transposed (head_dim-major) with its
// tokens XOR-swizzled in groups of four, so the MFMA operand reads are
// ds_read_b128 / ds_read_b64 with few bank conflicts.
//
// Waves own 16-row tiles of the query rows.  With RT <= 2 row tiles the four
// waves also split the tile's tokens (4/RT ways) and are combined through LDS
// at the end; with RT >= 4 every wave sees all tokens of its row tiles, so KV
// is read from HBM once per workgroup however many rows it serves.
//
// Scores: S^T = K Q^T with v_mfma_f32_16x16x32 (A = 8 consecutive head_dim
// elements of a token row, B = Q from registers).  The C layout of a 16-token
// S^T tile gives lane (lg, lc) tokens 4*lg..4*lg+3 of row lc, which is exactly
// the B operand (P^T) of v_mfma_f32_16x16x16 for O^T = V^T P^T, whose A
// operand is 4 consecutive tokens of one head_dim row of the transposed V.
constexpr int kTile = 64;              // tokens per LDS tile
constexpr int kMaxPagesLds = 1024;     // page ids of one item staged in LDS

template <int D>
struct TileLds {
  static constexpr int CPT = D / 8;                  // 16-byte chunks per token row
  static constexpr int K_BYTES = kTile * D * 2;
  static constexpr int V_BYTES = D * kTile * 2;
};

// V^T token swizzle: groups of four tokens are permuted per 8-row band of head_dim.
__device__ __forceinline__ int vt_swz(int d) { return (4 * (d >> 3)) & (kTile - 4); }

template <typename T, int D, int RT>
__global__ __launch_bounds__(256) void attn_tile_kernel(AttnArgs a) {
  constexpr int KS = D / 32;                         // QK contraction steps
  constexpr int MT = D / 16;                         // O^T head_dim tiles
  constexpr int CPT = D / 8;
  constexpr int LCH = kTile * CPT / 256;             // 16-byte chunks per thread per tile (K and V each)
  constexpr int NTW = RT <= 4 ? 1 : RT / 4;          // row tiles per wave
  constexpr int TSPLIT = RT >= 4 ? 1 : 4 / RT;       // waves sharing a row tile (token split)
  constexpr int STW = (kTile / 16) / TSPLIT;         // 16-token subtiles per wave per tile
  constexpr int KV_BYTES = TileLds<D>::K_BYTES + TileLds<D>::V_BYTES;
  constexpr int COMB_SLOT = (MT * 64 * 4 + 2 * 64) * 4;   // bytes: O^T frags + m + l of one wave
  static_assert(TSPLIT == 1 || (TSPLIT - 1) * RT * COMB_SLOT <= KV_BYTES, "combine scratch must fit");
  static_assert(LCH >= 1, "tile too small for the workgroup");

  if (a.live_items && (int)blockIdx.x >= *a.live_items) return;
  __shared__ __attribute__((aligned(16))) unsigned char kv_lds[KV_BYTES];
  __shared__ int pg_lds[kMaxPagesLds];
  uint16_t* kt = reinterpret_cast<uint16_t*>(kv_lds);
  uint16_t* vt = reinterpret_cast<uint16_t*>(kv_lds + TileLds<D>::K_BYTES);

  const WorkItem it = a.items[blockIdx.x];
  const int kvh = blockIdx.y;
  const int tid = threadIdx.x;
  const int w = tid >> 6, lane = tid & 63, lg = lane >> 4, lc = lane & 15;
  const int g = a.g, R = it.q_count * g, ps = a.page_size;
  const T* kv = reinterpret_cast<const T*>(a.kv);

  // ---- page ids of the item
  const int first_page = it.tok_begin / ps;
  const int n_pages = (it.tok_begin + it.tok_count - 1) / ps - first_page + 1;
  for (int i = tid; i < n_pages; i += 256) pg_lds[i] = a.pages[it.page_begin + first_page + i];

  // ---- wave role
  const int rt0 = (RT >= 4) ? w * NTW : (w % RT);
  const int ts = (RT >= 4) ? 0 : (w / RT);
  bool active[NTW];
  int lim[NTW];      // item tokens this lane's row sees (causal: its query's limit)
#pragma unroll
  for (int nt = 0; nt < NTW; ++nt) {
    active[nt] = (rt0 + nt) * 16 < R;
    const int64_t v = (int64_t)it.vis0 + ((rt0 + nt) * 16 + lc) / g - it.tok_begin;
    lim[nt] = (int)std::min<int64_t>(it.tok_count, std::max<int64_t>(v, 0));
  }

  // ---- Q as the B operand: lane holds Q[row = (rt0+nt)*16 + lc][d = ks*32 + 8*lg .. +7]
  v8s qf[NTW][KS];
#pragma unroll
  for (int nt = 0; nt < NTW; ++nt) {
    const int row = (rt0 + nt) * 16 + lc;
    if (row < R) {
      const int j = row / g, hh = row - j * g;
      const int qi = a.q_index[it.q_begin + j];
      const T* qp = reinterpret_cast<const T*>(a.q) + (int64_t)qi * a.q_sn + (int64_t)(kvh * g + hh) * a.q_sh;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) qf[nt][ks] = *reinterpret_cast<const v8s*>(qp + ks * 32 + lg * 8);
    } else {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) qf[nt][ks] = v8s{0, 0, 0, 0, 0, 0, 0, 0};
    }
  }
  __syncthreads();   // page ids staged

  // ---- tile loader: thread chunk c = i*256 + tid -> token c / CPT, column chunk c % CPT
  v8s kp[LCH], vp[LCH];
  auto load_tile = [&](int tile) {
#pragma unroll
    for (int i = 0; i < LCH; ++i) {
      const int c = i * 256 + tid;
      const int tl = tile * kTile + c / CPT;
      if (tl < it.tok_count) {
        const int tok = it.tok_begin + tl;
        const int page = pg_lds[tok / ps - first_page];
        const int64_t base = kv_off(page, 0, tok % ps, kvh, ps, a.hkv, D) + (c % CPT) * 8;
        const int64_t vstep = (int64_t)ps * a.hkv * D;     // K plane -> V plane of the page
        kp[i] = *reinterpret_cast<const v8s*>(kv + base);
        vp[i] = *reinterpret_cast<const v8s*>(kv + base + vstep);
      } else {
        kp[i] = v8s{0, 0, 0, 0, 0, 0, 0, 0};
        vp[i] = v8s{0, 0, 0, 0, 0, 0, 0, 0};
      }
    }
  };

  float m_run[NTW], l_run[NTW];
  v4f o_acc[NTW][MT];
#pragma unroll
  for (int nt = 0; nt < NTW; ++nt) {
    m_run[nt] = -INFINITY;
    l_run[nt] = 0.f;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) o_acc[nt][mt] = v4f{0.f, 0.f, 0.f, 0.f};
  }

  const int n_tiles = (it.tok_count + kTile - 1) / kTile;
  load_tile(0);
  for (int tile = 0; tile < n_tiles; ++tile) {
    __syncthreads();                                   // previous tile's LDS reads are done
#pragma unroll
    for (int i = 0; i < LCH; ++i) {
      const int c = i * 256 + tid;
      const int t = c / CPT, ch = c % CPT;
      *reinterpret_cast<v8s*>(kt + (t * CPT + (ch ^ (t & (CPT - 1)))) * 8) = kp[i];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int d = ch * 8 + e;
        vt[d * kTile + (t ^ vt_swz(d))] = (uint16_t)vp[i][e];
      }
    }
    __syncthreads();                                   // tile staged
    if (tile + 1 < n_tiles) load_tile(tile + 1);       // in flight during the compute below

    const int tl0 = tile * kTile;
#pragma unroll
    for (int nt = 0; nt < NTW; ++nt) {
      if (!active[nt]) continue;
      // scores of the wave's subtiles (lane: tokens 16*sub + 4*lg + r, row lc)
      float x[STW][4];
#pragma unroll
      for (int sb = 0; sb < STW; ++sb) {
        const int sub = ts * STW + sb;
        const int t = sub * 16 + lc;
        v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const int ch = ks * 4 + lg;
          const v8s kf = *reinterpret_cast<const v8s*>(kt + (t * CPT + (ch ^ (t & (CPT - 1)))) * 8);
          acc = mfma_qk<T>(kf, qf[nt][ks], acc);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int tl = tl0 + sub * 16 + 4 * lg + r;
          x[sb][r] = (tl < lim[nt]) ? acc[r] * a.scale_log2 : -INFINITY;
        }
      }
      float mx = -INFINITY;
#pragma unroll
      for (int sb = 0; sb < STW; ++sb)
#pragma unroll
        for (int r = 0; r < 4; ++r) mx = fmaxf(mx, x[sb][r]);
      mx = rows4_max(mx);
      const float m_new = fmaxf(m_run[nt], mx);
      const float msafe = (m_new == -INFINITY) ? 0.f : m_new;
      const float alpha = exp2f(m_run[nt] - msafe);    // 0 while nothing was seen
      float psum = 0.f;
      v4s pf[STW];
#pragma unroll
      for (int sb = 0; sb < STW; ++sb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float p = exp2f(x[sb][r] - msafe);
          psum += p;
          pf[sb][r] = (short)pack16<T>(p);
        }
      l_run[nt] = l_run[nt] * alpha + psum;
      m_run[nt] = m_new;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        v4f o = o_acc[nt][mt] * alpha;
#pragma unroll
        for (int sb = 0; sb < STW; ++sb) {
          const int d = mt * 16 + lc;
          const int tok = (ts * STW + sb) * 16 + 4 * lg;
          const v4s vf = *reinterpret_cast<const v4s*>(vt + d * kTile + (tok ^ vt_swz(d)));
          o = mfma_pv<T>(vf, pf[sb], o);
        }
        o_acc[nt][mt] = o;
      }
    }
  }

  // row sums over the four lane groups
#pragma unroll
  for (int nt = 0; nt < NTW; ++nt) {
    l_run[nt] = rows4_sum(l_run[nt]);
  }

  // ---- token-split waves (ts > 0) hand their state to the ts == 0 wave of the row tile
  if constexpr (TSPLIT > 1) {
    float* comb = reinterpret_cast<float*>(kv_lds);
    __syncthreads();                                   // tiles no longer needed
    if (ts > 0 && active[0]) {
      float* slot = comb + ((ts - 1) * RT + rt0) * (COMB_SLOT / 4);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) *reinterpret_cast<v4f*>(slot + (mt * 64 + lane) * 4) = o_acc[0][mt];
      slot[MT * 256 + lane] = m_run[0];
      slot[MT * 256 + 64 + lane] = l_run[0];
    }
    __syncthreads();
    if (ts == 0 && active[0]) {
#pragma unroll
      for (int s2 = 1; s2 < TSPLIT; ++s2) {
        const float* slot = comb + ((s2 - 1) * RT + rt0) * (COMB_SLOT / 4);
        const float mb = slot[MT * 256 + lane], lb = slot[MT * 256 + 64 + lane];
        const float M = fmaxf(m_run[0], mb);
        const float ca = (M == -INFINITY) ? 0.f : exp2f(m_run[0] - M);
        const float cb = (M == -INFINITY) ? 0.f : exp2f(mb - M);
        l_run[0] = l_run[0] * ca + lb * cb;
        m_run[0] = M;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          o_acc[0][mt] = o_acc[0][mt] * ca + *reinterpret_cast<const v4f*>(slot + (mt * 64 + lane) * 4) * cb;
      }
    }
  }

  // ---- writes: lane holds O^T[d = mt*16 + 4*lg + i][row = (rt0+nt)*16 + lc]
  if (ts == 0) {
#pragma unroll
    for (int nt = 0; nt < NTW; ++nt) {
      const int row = (rt0 + nt) * 16 + lc;
      if (!active[nt] || row >= R) continue;
      const int j = row / g, hh = row - j * g, head = kvh * g + hh;
      const float l = l_run[nt];
      const float inv = (l > 0.f) ? 1.f / l : 0.f;
      if (it.out_row < 0) {
        const int qi = a.q_index[it.q_begin + j];
        T* op = reinterpret_cast<T*>(a.out) + (int64_t)qi * a.o_sn + (int64_t)head * a.o_sh;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          v4s pk;
#pragma unroll
          for (int i = 0; i < 4; ++i) pk[i] = (short)pack16<T>(o_acc[nt][mt][i] * inv);
          *reinterpret_cast<v4s*>(op + mt * 16 + 4 * lg) = pk;
        }
      } else {
        float* op = a.part_o + ((int64_t)(it.out_row + j) * a.hq + head) * D;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) *reinterpret_cast<v4f*>(op + mt * 16 + 4 * lg) = o_acc[nt][mt] * inv;
      }
      if (lg == 0) store_row_lse<T>(a, it, j, head, m_run[nt], l);
    }
  }
  __shared__ int s_last[kMaxTileRows];
  if (it.out_row >= 0 && a.counters) fused_merge_epilogue<T, D>(a, it, kvh, s_last);
}

// ================================================================== VALU kernel
// Any storage dtype, D in {64, 128, 256}, up to 32 rows per tile.  K/V blocks
// of 32 tokens are converted to fp32 in LDS; scores use one thread per
// (token, row-group), P.V one thread per (head_dim column, row-group).
template <typename T, int D>
__global__ __launch_bounds__(256) void attn_valu_kernel(AttnArgs a) {
  constexpr int BT = 32;
  constexpr int NRG = 256 / D;           // row groups in the P.V phase
  constexpr int RPT = kMaxRows / NRG;    // rows per thread in the P.V phase
  constexpr int KST = D + 1;             // padded K row
  __shared__ float qs[kMaxRows][D];
  __shared__ float ks[BT * KST];
  __shared__ float vs[BT][D];
  __shared__ float psm[kMaxRows][BT];
  __shared__ float alpha_s[kMaxRows], l_s[kMaxRows], m_s[kMaxRows];
  if (a.live_items && (int)blockIdx.x >= *a.live_items) return;

  const WorkItem it = a.items[blockIdx.x];
  const int kvh = blockIdx.y;
  const int tid = threadIdx.x;
  const int g = a.g;
  const int R = it.q_count * g;
  const T* qbase = reinterpret_cast<const T*>(a.q);
  const T* kv = reinterpret_cast<const T*>(a.kv);
  const int ps = a.page_size;

  for (int e = tid; e < kMaxRows * D; e += 256) {
    const int r = e / D, d = e % D;
    float val = 0.f;
    if (r < R) {
      const int j = r / g, hh = r - j * g;
      const int qi = a.q_index[it.q_begin + j];
      val = to_f32(qbase[(int64_t)qi * a.q_sn + (int64_t)(kvh * g + hh) * a.q_sh + d]);
    }
    qs[r][d] = val;
  }

  // score-phase ownership: token t = tid % 32, rows rg + 8k
  const int t_own = tid & 31, rg = tid >> 5;
  float m_row[4], l_row[4];
  int lim_row[4];    // item tokens row rg + 8k sees (causal: its query's limit)
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    m_row[k] = -INFINITY;
    l_row[k] = 0.f;
    const int64_t v = (int64_t)it.vis0 + (rg + 8 * k) / g - it.tok_begin;
    lim_row[k] = (int)std::min<int64_t>(it.tok_count, std::max<int64_t>(v, 0));
  }
  // P.V-phase ownership: column d = tid % D, rows rgp + NRG*k
  const int d_own = tid % D, rgp = tid / D;
  float acc[RPT];
#pragma unroll
  for (int k = 0; k < RPT; ++k) acc[k] = 0.f;

  for (int tb = 0; tb < it.tok_count; tb += BT) {
    __syncthreads();
    for (int e = tid; e < BT * D; e += 256) {
      const int t = e / D, d = e % D;
      const int tl = tb + t;
      float kx = 0.f, vx = 0.f;
      if (tl < it.tok_count) {
        const int tok = it.tok_begin + tl;
        const int page = a.pages[it.page_begin + tok / ps];
        kx = to_f32(kv[kv_off(page, 0, tok % ps, kvh, ps, a.hkv, D) + d]);
        vx = to_f32(kv[kv_off(page, 1, tok % ps, kvh, ps, a.hkv, D) + d]);
      }
      ks[t * KST + d] = kx;
      vs[t][d] = vx;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int r = rg + 8 * k;
      float sc = 0.f;
#pragma unroll 8
      for (int d = 0; d < D; ++d) sc += qs[r][d] * ks[t_own * KST + d];
      const float x = (tb + t_own) < lim_row[k] ? sc * a.scale_log2 : -INFINITY;
      float mx = x;
#pragma unroll
      for (int o = 16; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
      const float m_new = fmaxf(m_row[k], mx);
      const float msafe = (m_new == -INFINITY) ? 0.f : m_new;   // a row with nothing seen yet
      const float p = exp2f(x - msafe);
      float psum = p;
#pragma unroll
      for (int o = 16; o > 0; o >>= 1) psum += __shfl_xor(psum, o, 64);
      const float al = exp2f(m_row[k] - msafe);
      l_row[k] = l_row[k] * al + psum;
      m_row[k] = m_new;
      psm[r][t_own] = p;
      if (t_own == 0) alpha_s[r] = al;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
      const int r = rgp + NRG * k;
      float sacc = acc[k] * alpha_s[r];
#pragma unroll 8
      for (int t = 0; t < BT; ++t) sacc += psm[r][t] * vs[t][d_own];
      acc[k] = sacc;
    }
  }
  if (t_own == 0) {
#pragma unroll
    for (int k = 0; k < 4; ++k) { l_s[rg + 8 * k] = l_row[k]; m_s[rg + 8 * k] = m_row[k]; }
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < RPT; ++k) {
    const int r = rgp + NRG * k;
    if (r >= R) continue;
    const int j = r / g, hh = r - j * g, head = kvh * g + hh;
    const float l = l_s[r];
    const float o = (l > 0.f) ? acc[k] / l : 0.f;
    if (it.out_row < 0) {
      const int qi = a.q_index[it.q_begin + j];
      reinterpret_cast<T*>(a.out)[(int64_t)qi * a.o_sn + (int64_t)head * a.o_sh + d_own] = from_f32<T>(o);
    } else {
      a.part_o[((int64_t)(it.out_row + j) * a.hq + head) * D + d_own] = o;
    }
    if (d_own == 0) store_row_lse<T>(a, it, j, head, m_s[r], l);
  }
  __shared__ int s_last[kMaxRows];
  if (it.out_row >= 0 && a.counters) fused_merge_epilogue<T, D>(a, it, kvh, s_last);
}

// ================================================================== merge kernel
// One workgroup per merged query: the lse of every (partial row, head) pair is
// read in parallel and turned into normalised weights in LDS, then every
// thread accumulates 4 consecutive head_dim columns of one head over the rows
// (independent loads, no dependent chain).
constexpr int kMergeMaxRows = 64;

template <typename T, int D>
__global__ __launch_bounds__(256) void merge_kernel(MergeArgs a) {
  __shared__ float wgt[kMergeMaxRows * kMaxTileRows];   // [row][head] weights
  __shared__ int rows_s[kMergeMaxRows];
  __shared__ float lse_h[kMaxTileRows];
  if (a.live && (int)blockIdx.x >= *a.live) return;
  const int tid = threadIdx.x;
  const int qi = a.merge_q[blockIdx.x];
  const int b = a.merge_ptr[blockIdx.x], e = a.merge_ptr[blockIdx.x + 1];
  const int hq = a.hq;
  T* out = reinterpret_cast<T*>(a.out) + (int64_t)qi * a.o_sn;
  if (e - b > kMergeMaxRows || hq > kMaxTileRows) {
    // long merges: one wave per head, sequential over rows
    for (int head = tid >> 6; head < hq; head += 4) {
      const int lane = tid & 63;
      float M = -INFINITY;
      for (int i = b; i < e; ++i) M = fmaxf(M, a.part_lse[(int64_t)a.merge_rows[i] * hq + head]);
      float z = 0.f, acc[D / 64];
#pragma unroll
      for (int k = 0; k < D / 64; ++k) acc[k] = 0.f;
      if (M != -INFINITY)
        for (int i = b; i < e; ++i) {
          const int64_t row = (int64_t)a.merge_rows[i] * hq + head;
          const float w = expf(a.part_lse[row] - M);
          z += w;
#pragma unroll
          for (int k = 0; k < D / 64; ++k) acc[k] += w * a.part_o[row * D + lane + 64 * k];
        }
      const float inv = (z > 0.f) ? 1.f / z : 0.f;
#pragma unroll
      for (int k = 0; k < D / 64; ++k) out[(int64_t)head * a.o_sh + lane + 64 * k] = from_f32<T>(acc[k] * inv);
      if (a.out_lse && lane == 0) a.out_lse[(int64_t)qi * hq + head] = (z > 0.f) ? M + logf(z) : -INFINITY;
    }
    return;
  }
  const int nr = e - b;
  for (int i = tid; i < nr; i += 256) rows_s[i] = a.merge_rows[b + i];
  __syncthreads();
  for (int i = tid; i < nr * hq; i += 256) {
    const int r = i / hq, h = i - r * hq;
    wgt[r * hq + h] = a.part_lse[(int64_t)rows_s[r] * hq + h];
  }
  __syncthreads();
  for (int h = tid; h < hq; h += 256) {
    float M = -INFINITY;
    for (int r = 0; r < nr; ++r) M = fmaxf(M, wgt[r * hq + h]);
    float z = 0.f;
    if (M != -INFINITY)
      for (int r = 0; r < nr; ++r) z += expf(wgt[r * hq + h] - M);
    const float inv = (z > 0.f) ? 1.f / z : 0.f;
    for (int r = 0; r < nr; ++r) wgt[r * hq + h] = (M != -INFINITY) ? expf(wgt[r * hq + h] - M) * inv : 0.f;
    lse_h[h] = (z > 0.f) ? M + logf(z) : -INFINITY;
  }
  __syncthreads();
  constexpr int C4 = D / 4;                       // float4 columns per head
  for (int i = tid; i < hq * C4; i += 256) {
    const int h = i / C4, c = i - h * C4;
    v4f acc = {0.f, 0.f, 0.f, 0.f};
    for (int r = 0; r < nr; ++r) {
      const v4f o = *reinterpret_cast<const v4f*>(a.part_o + ((int64_t)rows_s[r] * hq + h) * D + 4 * c);
      acc += o * wgt[r * hq + h];
    }
    T* op = out + (int64_t)h * a.o_sh + 4 * c;
#pragma unroll
    for (int k = 0; k < 4; ++k) op[k] = from_f32<T>(acc[k]);
  }
  if (a.out_lse)
    for (int h = tid; h < hq; h += 256) a.out_lse[(int64_t)qi * hq + h] = lse_h[h];
}

// One wave owns one row, so outputs may alias inputs (every lane reads the
// row's lse before lane 0 overwrites it).
__global__ __launch_bounds__(256) void merge2_kernel(const float* oa, const float* la, const float* ob,
                                                    const float* lb, float* oo, float* lo, int rows,
                                                    int d) {
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= rows) return;
  const float x = la[r], y = lb[r];
  const float M = fmaxf(x, y);
  float ca = 0.f, cb = 0.f;
  if (M != -INFINITY) { ca = expf(x - M); cb = expf(y - M); }
  const float z = ca + cb;
  const float inv = (z > 0.f) ? 1.f / z : 0.f;
  for (int e = lane; e < d; e += 64) {
    const int64_t i = r * d + e;
    oo[i] = (ca * oa[i] + cb * ob[i]) * inv;
  }
  if (lane == 0) lo[r] = (z > 0.f) ? M + logf(z) : -INFINITY;
}

// ================================================================== host: planner
int attn_plan(const be_level* levels, int num_levels, int num_queries, int hq, int hkv, int d,
              int page_size, int num_pages, int dtype, int flags, int num_cus, const be_plan_caps* caps,
              int32_t* out, int64_t cap, be_attn_plan_info* info) {
  BE_REQUIRE(info != nullptr && out != nullptr, "null plan buffer or info");
  memset(info, 0, sizeof(*info));
  BE_REQUIRE(num_levels >= 0 && (num_levels == 0 || levels != nullptr), "bad levels");
  BE_REQUIRE(num_queries >= 0, "num_queries must be >= 0");
  BE_REQUIRE(hq > 0 && hkv > 0 && hq % hkv == 0, "num_qo_heads (%d) must be a multiple of num_kv_heads (%d)", hq, hkv);
  BE_REQUIRE(page_size > 0 && num_pages > 0, "page_size and num_pages must be positive");
  BE_REQUIRE(dtype == BE_F32 || dtype == BE_F16 || dtype == BE_BF16, "unknown dtype %d", dtype);
  const int g = hq / hkv;
  if (d != 64 && d != 128 && d != 256) return fail(BE_ERR_UNSUPPORTED, "head_dim %d: kernels exist for 64, 128, 256", d);
  if (g > kMaxTileRows) return fail(BE_ERR_UNSUPPORTED, "GQA group %d exceeds %d", g, kMaxTileRows);
  if (num_cus <= 0) num_cus = 256;

  // ---- validate levels, collect groups
  std::vector<Group> groups;
  {
    int64_t ng = 0;
    for (int lv = 0; lv < num_levels; ++lv) ng += std::max(0, levels[lv].num_groups);
    groups.reserve((size_t)ng);
  }
  int64_t total_pages = 0;
  for (int lv = 0; lv < num_levels; ++lv) {
    const be_level& L = levels[lv];
    BE_REQUIRE(L.num_groups >= 0, "level %d: negative group count", lv);
    BE_REQUIRE(L.num_groups == 0 || (L.qo_indptr && L.kv_indptr && L.last_page_len), "level %d: null index array", lv);
    if (L.num_groups == 0) continue;
    BE_REQUIRE(L.qo_indptr[0] == 0 && L.kv_indptr[0] == 0, "level %d: indptr must start at 0", lv);
    for (int j = 0; j < L.num_groups; ++j) {
      BE_REQUIRE(L.qo_indptr[j + 1] >= L.qo_indptr[j], "level %d: qo_indptr not monotone", lv);
      BE_REQUIRE(L.kv_indptr[j + 1] >= L.kv_indptr[j], "level %d: kv_indptr not monotone", lv);
      BE_REQUIRE(L.last_page_len[j] >= 0 && L.last_page_len[j] <= page_size,
                 "level %d group %d: last_page_len %d outside [0, %d]", lv, j, L.last_page_len[j], page_size);
    }
    BE_REQUIRE(L.qo_indptr[L.num_groups] <= num_queries, "level %d: qo_indptr exceeds %d queries", lv, num_queries);
    const int np = L.kv_indptr[L.num_groups];
    BE_REQUIRE(np == 0 || L.kv_indices, "level %d: null kv_indices", lv);
    for (int i = 0; i < np; ++i)
      BE_REQUIRE(L.kv_indices[i] >= 0 && L.kv_indices[i] < num_pages, "level %d: page %d out of range [0, %d)", lv,
                 L.kv_indices[i], num_pages);
    for (int j = 0; j < L.num_groups; ++j) {
      const int npg = L.kv_indptr[j + 1] - L.kv_indptr[j];
      const int kv_len = npg == 0 ? 0 : (npg - 1) * page_size + L.last_page_len[j];
      groups.push_back(Group{lv, L.qo_indptr[j], L.qo_indptr[j + 1], (int)(total_pages + L.kv_indptr[j]), kv_len});
    }
    total_pages += np;
  }

  // ---- algorithmic bytes: distinct (page, head) valid tokens, plus Q and O
  // (a per-thread table of the pool's pages, zero between calls: only the
  // referenced entries are set, summed and cleared)
  static thread_local std::vector<int> valid;
  if ((int)valid.size() < num_pages) valid.assign((size_t)num_pages, 0);
  for (int lv = 0; lv < num_levels; ++lv) {
    const be_level& L = levels[lv];
    for (int j = 0; j < L.num_groups; ++j) {
      const int b = L.kv_indptr[j], e = L.kv_indptr[j + 1];
      for (int i = b; i < e; ++i) {
        const int v = (i + 1 < e) ? page_size : L.last_page_len[j];
        int& slot = valid[L.kv_indices[i]];
        slot = std::max(slot, v);
      }
    }
  }
  int64_t valid_tokens = 0;
  for (int lv = 0; lv < num_levels; ++lv) {
    const be_level& L = levels[lv];
    const int np = L.num_groups ? L.kv_indptr[L.num_groups] : 0;
    for (int i = 0; i < np; ++i) {
      valid_tokens += valid[L.kv_indices[i]];
      valid[L.kv_indices[i]] = 0;
    }
  }
  const int64_t es = (int64_t)dtype_size(dtype);
  double flops = 0.0;
  // causal (BE_PLAN_CAUSAL): on the last level, query q0 + i of a group of n
  // queries sees its first kv_len - n + i + 1 tokens (FlashInfer's alignment of
  // the query block to the end of the keys; one query per group masks nothing)
  const bool causal = (flags & BE_PLAN_CAUSAL) != 0;
  auto is_causal = [&](const Group& gr) { return causal && gr.level == num_levels - 1 && gr.q1 - gr.q0 > 1; };
  auto vis = [&](const Group& gr, int qi) -> int {
    if (!is_causal(gr)) return gr.kv_len;
    return std::max(0, std::min(gr.kv_len, gr.kv_len - (gr.q1 - gr.q0) + (qi - gr.q0) + 1));
  };
  bool any_causal = false;
  for (const Group& gr : groups) {
    if (gr.kv_len <= 0 || gr.q1 <= gr.q0) continue;
    any_causal = any_causal || is_causal(gr);
    if (is_causal(gr)) {
      for (int qi = gr.q0; qi < gr.q1; ++qi) flops += 4.0 * d * hq * (double)vis(gr, qi);
    } else {
      flops += 4.0 * d * hq * (double)gr.kv_len * (gr.q1 - gr.q0);
    }
  }

  bool mfma = (dtype != BE_F32) && !(flags & BE_PLAN_FORCE_VALU);
  if (!mfma && g > kMaxRows) return fail(BE_ERR_UNSUPPORTED, "GQA group %d exceeds %d (VALU kernel)", g, kMaxRows);
  if (mfma && d == 256 && g > 64) return fail(BE_ERR_UNSUPPORTED, "GQA group %d exceeds 64 at head_dim 256", g);
  // rows per workgroup: MFMA 8 row tiles (4 at head_dim 256, VGPR budget), VALU 32
  int rows_cap = mfma ? (d == 256 ? 64 : kMaxTileRows) : kMaxRows;
  if (caps) {
    BE_REQUIRE(!(flags & BE_PLAN_FUSED_MERGE), "the fused merge is not available with a fixed-capacity layout");
    const int tr = caps->tile_rows;
    BE_REQUIRE(tr == 16 || tr == 32 || tr == 64 || tr == 128, "caps.tile_rows must be 16, 32, 64 or 128");
    BE_REQUIRE(tr >= g, "caps.tile_rows %d smaller than the GQA group %d", tr, g);
    BE_REQUIRE(caps->max_items >= 0 && caps->max_queries >= num_queries && caps->max_pages >= 0 &&
                   caps->max_merge >= 0 && caps->max_merge_rows >= 0 && caps->max_zero >= 0,
               "bad plan capacities (max_queries %d < %d queries?)", caps->max_queries, num_queries);
    if (mfma) rows_cap = std::min(rows_cap, tr);
  }
  // merge-free row blocks (decode plans, compact layout): forced by
  // BE_PLAN_ROWS, else chosen when rows_preferred says so
  bool rows_ok = false;
  if (!any_causal && !caps && stream_eligible(dtype, d, g, page_size, flags) && g <= 16 &&
      !(flags & BE_PLAN_NO_ROWS) && ((flags & BE_PLAN_ROWS) || rows_preferred(groups, num_queries, g, num_cus))) {
    memset(info, 0, sizeof(*info));
    const int rc = rows_plan(groups, levels, num_levels, total_pages, num_queries, hq, hkv, page_size, num_cus, out,
                             cap, info);
    if (rc != BE_OK && rc != BE_ERR_UNSUPPORTED) return rc;
    rows_ok = rc == BE_OK;     // unsupported: a task exceeds the kernel's LDS tables
  }
  if (rows_ok) {
    info->num_qo_heads = hq;
    info->num_kv_heads = hkv;
    info->head_dim = d;
    info->page_size = page_size;
    info->num_pages = num_pages;
    info->dtype = dtype;
    info->kv_bytes = valid_tokens * hkv * d * es * 2;
    info->qo_bytes = (int64_t)num_queries * hq * d * es * 2;
    info->flops = flops;
    return BE_OK;
  }
  if (!(any_causal && caps) && stream_eligible(dtype, d, g, page_size, flags) && (!caps || caps->tile_rows == 64)) {
    memset(info, 0, sizeof(*info));
    const int rc = stream_plan(groups, levels, num_levels, total_pages, num_queries, hq, hkv, d, page_size,
                               num_pages, dtype, num_cus, flags, caps, out, cap, info);
    if (rc == BE_OK) {
      info->num_qo_heads = hq;
      info->num_kv_heads = hkv;
      info->head_dim = d;
      info->page_size = page_size;
      info->num_pages = num_pages;
      info->dtype = dtype;
      info->kv_bytes = valid_tokens * hkv * d * es * 2;
      info->qo_bytes = (int64_t)num_queries * hq * d * es * 2;
      info->flops = flops;
      return BE_OK;
    }
    if (rc != BE_ERR_UNSUPPORTED) return rc;
    // a workgroup would need more segments than its table holds: tile kernel
  }
  const int q_tile = std::max(1, rows_cap / g);

  // ---- split-K chunk: about two workgroups per CU over all (tile, chunk, head)
  int64_t work = 0;   // token-tiles
  for (const Group& gr : groups)
    if (gr.q1 > gr.q0 && gr.kv_len > 0) work += ceil_div(gr.q1 - gr.q0, q_tile) * (int64_t)gr.kv_len;
  const int64_t target = 3 * (int64_t)num_cus;
  int64_t chunk = ceil_div(work * hkv, target);
  chunk = std::max<int64_t>(128, ceil_div(chunk, 64) * 64);
  // an item's page ids are staged in LDS: at most kMaxPagesLds pages per item
  const int64_t chunk_cap = std::max<int64_t>(64, ((int64_t)(kMaxPagesLds - 1) * page_size) / 64 * 64);
  if (chunk > chunk_cap) chunk = chunk_cap;

  // A chunk of a group writes rows x D x 4 bytes of partials per KV head while
  // reading 4 x D bytes per token (bf16 K + V): keep chunks >= 4 x rows tokens
  // so partial traffic stays under ~1/4 of the KV bytes it summarises.
  auto group_chunk = [&](const Group& gr) -> int64_t {
    const int64_t rows = (int64_t)std::min(q_tile, gr.q1 - gr.q0) * g;
    int64_t c = std::max<int64_t>(chunk, ceil_div(4 * rows, 64) * 64);
    return std::min(c, chunk_cap);
  };

  // ---- per-query partial counts (a causal query tile stops at the chunk
  // holding its last query's last visible token)
  std::vector<int> cnt(num_queries, 0);
  for (const Group& gr : groups) {
    if (gr.kv_len <= 0 || gr.q1 <= gr.q0) continue;
    const int64_t gchunk = group_chunk(gr);
    for (int qa = gr.q0; qa < gr.q1; qa += q_tile) {
      const int qn = std::min(q_tile, gr.q1 - qa);
      const int nch = (int)ceil_div(vis(gr, qa + qn - 1), gchunk);
      for (int qi = qa; qi < qa + qn; ++qi) cnt[qi] += nch;
    }
  }

  // ---- items and partial rows
  std::vector<WorkItem> items;
  std::vector<std::vector<int>> rows_of(num_queries);
  int rows = 0, max_r = 0;
  for (const Group& gr : groups) {
    if (gr.kv_len <= 0 || gr.q1 <= gr.q0) continue;
    const int64_t gchunk = group_chunk(gr);
    for (int t0 = 0; t0 < gr.kv_len; t0 += (int)gchunk) {
      for (int qa = gr.q0; qa < gr.q1; qa += q_tile) {
        const int qn = std::min(q_tile, gr.q1 - qa);
        const int tile_vis = vis(gr, qa + qn - 1);     // the tile's last query sees the most
        if (t0 >= tile_vis) continue;
        const int tc = (int)std::min<int64_t>(gchunk, tile_vis - t0);
        bool direct = true;
        for (int qi = qa; qi < qa + qn; ++qi) direct = direct && (cnt[qi] == 1);
        // vis0: tokens the item's first query sees (group token units, before
        // clamping to [0, kv_len]: may be negative), query j of the item sees
        // vis0 + j (the kernel clamps per row); kNoCausal without the mask
        const int vis0 = gr.kv_len - (gr.q1 - gr.q0) + (qa - gr.q0) + 1;
        WorkItem w{qa, qn, gr.page_base, t0, tc, -1, is_causal(gr) ? vis0 : kNoCausal, 0};
        if (!direct) {
          w.out_row = rows;
          for (int j = 0; j < qn; ++j) rows_of[qa + j].push_back(rows + j);
          rows += qn;
        }
        max_r = std::max(max_r, qn * g);
        items.push_back(w);
      }
    }
  }

  // ---- merge list (queries with >= 2 partial rows) and zero list (no keys)
  std::vector<int> merge_q, merge_ptr{0}, merge_rows, zero_q;
  for (int qi = 0; qi < num_queries; ++qi) {
    if (cnt[qi] == 1) continue;
    if (cnt[qi] == 0) {
      zero_q.push_back(qi);
      continue;
    }
    merge_q.push_back(qi);
    for (int r : rows_of[qi]) merge_rows.push_back(r);
    merge_ptr.push_back((int)merge_rows.size());
  }

  // ---- serialise: header of live counts, then the regions (sized to this
  //      plan, or to the capacities of a fixed layout)
  const int64_t n_items = (int64_t)items.size();
  if (caps) {
    if (n_items > caps->max_items || total_pages > caps->max_pages || (int64_t)merge_q.size() > caps->max_merge ||
        rows > caps->max_merge_rows || (int64_t)zero_q.size() > caps->max_zero)
      return fail(BE_ERR_CAPACITY,
                  "plan exceeds its fixed capacities: items %lld/%d pages %lld/%d merge %zu/%d rows %d/%d zero %zu/%d",
                  (long long)n_items, caps->max_items, (long long)total_pages, caps->max_pages, merge_q.size(),
                  caps->max_merge, rows, caps->max_merge_rows, zero_q.size(), caps->max_zero);
  }
  const int64_t c_items = caps ? caps->max_items : n_items;
  const int64_t c_q = caps ? caps->max_queries : num_queries;
  const int64_t c_pages = caps ? caps->max_pages : total_pages;
  const int64_t c_merge = caps ? caps->max_merge : (int64_t)merge_q.size();
  const int64_t c_rows = caps ? caps->max_merge_rows : (int64_t)merge_rows.size();
  const int64_t c_zero = caps ? caps->max_zero : (int64_t)zero_q.size();
  int64_t off = kPlanHeader;
  const int64_t off_items = off;    off += c_items * 8;
  const int64_t off_qindex = off;   off += c_q;
  const int64_t off_pages = off;    off += c_pages;
  const int64_t off_mq = off;       off += c_merge;
  const int64_t off_mp = off;       off += c_merge + 1;
  const int64_t off_mr = off;       off += c_rows;
  const int64_t off_qm = off;       off += c_q;
  const int64_t off_zq = off;       off += c_zero;
  const int64_t off_zp = off;       off += c_zero + 1;
  off = ceil_div(off, 4) * 4;
  if (off > cap || off > INT32_MAX) {
    info->plan_ints = (int32_t)std::min<int64_t>(off, INT32_MAX);   // the words needed (0: a capacity of caps)
    return fail(BE_ERR_CAPACITY, "plan needs %lld int32 words, buffer holds %lld", (long long)off, (long long)cap);
  }
  for (int i = 0; i < kPlanHeader; ++i) out[i] = 0;
  out[kHdrItems] = (int32_t)n_items;
  out[kHdrMerge] = (int32_t)merge_q.size();
  out[kHdrZero] = (int32_t)zero_q.size();
  out[kHdrRows] = rows;
  memcpy(out + off_items, items.data(), n_items * sizeof(WorkItem));
  for (int i = 0; i < num_queries; ++i) out[off_qindex + i] = i;
  {
    int64_t p = off_pages;
    for (int lv = 0; lv < num_levels; ++lv) {
      const be_level& L = levels[lv];
      const int np = L.num_groups ? L.kv_indptr[L.num_groups] : 0;
      if (np) memcpy(out + p, L.kv_indices, np * sizeof(int32_t));
      p += np;
    }
  }
  if (!merge_q.empty()) memcpy(out + off_mq, merge_q.data(), merge_q.size() * 4);
  memcpy(out + off_mp, merge_ptr.data(), merge_ptr.size() * 4);
  if (!merge_rows.empty()) memcpy(out + off_mr, merge_rows.data(), merge_rows.size() * 4);
  for (int qi = 0; qi < num_queries; ++qi) out[off_qm + qi] = -1;
  for (size_t m = 0; m < merge_q.size(); ++m) out[off_qm + merge_q[m]] = (int32_t)m;
  if (!zero_q.empty()) memcpy(out + off_zq, zero_q.data(), zero_q.size() * 4);
  for (int64_t i = off_zp; i < off_zp + (int64_t)zero_q.size() + 1; ++i) out[i] = 0;   // zero_ptr: empty ranges

  memset(info, 0, sizeof(*info));
  info->num_items = (int32_t)n_items;
  info->num_part_rows = rows;
  info->num_merge = (int32_t)merge_q.size();
  info->num_queries = num_queries;
  info->num_qo_heads = hq;
  info->num_kv_heads = hkv;
  info->head_dim = d;
  info->page_size = page_size;
  info->num_pages = num_pages;
  info->dtype = dtype;
  info->kernel = mfma ? 1 : 0;
  info->tile_rows = caps ? caps->tile_rows : (max_r <= 16 ? 16 : max_r <= 32 ? 32 : max_r <= 64 ? 64 : 128);
  info->chunk_tokens = (int32_t)std::min<int64_t>(chunk, INT32_MAX);
  info->plan_ints = (int32_t)off;
  info->off_items = (int32_t)off_items;
  info->off_qindex = (int32_t)off_qindex;
  info->off_pages = (int32_t)off_pages;
  info->off_merge_q = (int32_t)off_mq;
  info->off_merge_ptr = (int32_t)off_mp;
  info->off_merge_rows = (int32_t)off_mr;
  info->off_q_merge = (int32_t)off_qm;
  info->fused_merge = (flags & BE_PLAN_FUSED_MERGE) ? 1 : 0;
  info->num_zero = (int32_t)zero_q.size();
  info->off_zero_q = (int32_t)off_zq;
  info->off_zero_ptr = (int32_t)off_zp;
  info->static_layout = caps ? 1 : 0;
  info->grid_items = (int32_t)c_items;
  info->grid_merge = (int32_t)c_merge;
  info->grid_zero = (int32_t)c_zero;
  info->part_rows_cap = (int32_t)(caps ? caps->max_merge_rows : rows);
  info->counter_offset = ceil_div((int64_t)info->part_rows_cap * hq * (d + 1) * 4, 256) * 256;
  info->counter_bytes = info->fused_merge ? (int64_t)merge_q.size() * hkv * 4 : 0;
  info->partial_bytes = info->counter_offset + info->counter_bytes;
  info->kv_bytes = valid_tokens * hkv * d * es * 2;
  info->qo_bytes = (int64_t)num_queries * hq * d * es * 2;
  info->flops = flops;
  return BE_OK;
}

// ================================================================== host: run
template <typename T>
static int launch_attn(const be_attn_plan_info* info, AttnArgs& a, hipStream_t st) {
  const dim3 grid(info->grid_items, info->num_kv_heads);
  if (info->kernel == 1) {
    if constexpr (sizeof(T) == 2) {
      const int rt = info->tile_rows / 16;
#define BE_TILE_LAUNCH(DD)                                                                    \
  switch (rt) {                                                                               \
    case 1: attn_tile_kernel<T, DD, 1><<<grid, 256, 0, st>>>(a); break;                       \
    case 2: attn_tile_kernel<T, DD, 2><<<grid, 256, 0, st>>>(a); break;                       \
    case 4: attn_tile_kernel<T, DD, 4><<<grid, 256, 0, st>>>(a); break;                       \
    case 8: if (DD == 256) return fail(BE_ERR_UNSUPPORTED, "128-row tiles at head_dim 256"); \
            attn_tile_kernel<T, DD, (DD == 256 ? 4 : 8)><<<grid, 256, 0, st>>>(a); break;     \
    default: return fail(BE_ERR_INVALID, "corrupt plan: tile_rows %d", info->tile_rows);      \
  }
      switch (info->head_dim) {
        case 64: BE_TILE_LAUNCH(64) break;
        case 128: BE_TILE_LAUNCH(128) break;
        case 256: BE_TILE_LAUNCH(256) break;
        default: return fail(BE_ERR_UNSUPPORTED, "head_dim %d", info->head_dim);
      }
#undef BE_TILE_LAUNCH
    } else {
      return fail(BE_ERR_UNSUPPORTED, "MFMA kernel needs fp16/bf16 storage");
    }
  } else {
    switch (info->head_dim) {
      case 64: attn_valu_kernel<T, 64><<<grid, 256, 0, st>>>(a); break;
      case 128: attn_valu_kernel<T, 128><<<grid, 256, 0, st>>>(a); break;
      case 256: attn_valu_kernel<T, 256><<<grid, 256, 0, st>>>(a); break;
      default: return fail(BE_ERR_UNSUPPORTED, "head_dim %d", info->head_dim);
    }
  }
  BE_HIP_CHECK(hipGetLastError());
  return BE_OK;
}

template <typename T>
static int launch_merge(const be_attn_plan_info* info, MergeArgs& m, int count, hipStream_t st) {
  const dim3 grid(count);
  switch (info->head_dim) {
    case 64: merge_kernel<T, 64><<<grid, 256, 0, st>>>(m); break;
    case 128: merge_kernel<T, 128><<<grid, 256, 0, st>>>(m); break;
    case 256: merge_kernel<T, 256><<<grid, 256, 0, st>>>(m); break;
    default: return fail(BE_ERR_UNSUPPORTED, "head_dim %d", info->head_dim);
  }
  BE_HIP_CHECK(hipGetLastError());
  return BE_OK;
}

int attn_run(const be_attn_plan_info* info, const int32_t* plan, void* partials, const void* q,
             int64_t q_sn, int64_t q_sh, const void* kv, void* out, int64_t o_sn, int64_t o_sh,
             float* lse, float sm_scale, int phases, void* stream) {
  BE_REQUIRE(phases >= 1 && phases <= 3, "phases must be a non-empty subset of attention | merge");
  BE_REQUIRE(info && plan, "null plan");
  BE_REQUIRE(q && kv && out, "null q / kv / out");
  BE_REQUIRE(info->part_rows_cap == 0 || partials, "plan needs %lld bytes of partial scratch", (long long)info->partial_bytes);
  BE_REQUIRE(info->num_qo_heads % info->num_kv_heads == 0, "corrupt plan info");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (info->kernel == 2)
    return stream_run(info, plan, partials, q, q_sn, q_sh, kv, out, o_sn, o_sh, lse, sm_scale, phases, st);
  if (info->kernel == 3) return rows_run(info, plan, q, q_sn, q_sh, kv, out, o_sn, o_sh, lse, sm_scale, phases, st);
  const int64_t rows = info->part_rows_cap;
  AttnArgs a;
  a.q = q; a.q_sn = q_sn; a.q_sh = q_sh;
  a.kv = kv; a.out = out; a.o_sn = o_sn; a.o_sh = o_sh; a.out_lse = lse;
  a.part_o = reinterpret_cast<float*>(partials);
  a.part_lse = a.part_o + rows * info->num_qo_heads * info->head_dim;
  a.items = reinterpret_cast<const WorkItem*>(plan + info->off_items);
  a.q_index = plan + info->off_qindex;
  a.pages = plan + info->off_pages;
  a.page_size = info->page_size;
  a.hkv = info->num_kv_heads;
  a.hq = info->num_qo_heads;
  a.g = info->num_qo_heads / info->num_kv_heads;
  a.scale_log2 = sm_scale * 1.4426950408889634f;
  a.q_merge = plan + info->off_q_merge;
  a.merge_ptr = plan + info->off_merge_ptr;
  a.merge_rows = plan + info->off_merge_rows;
  a.live_items = info->static_layout ? plan + kHdrItems : nullptr;
  a.counters = (info->fused_merge && info->num_merge > 0)
                   ? reinterpret_cast<int32_t*>(reinterpret_cast<char*>(partials) + info->counter_offset)
                   : nullptr;
  int rc = BE_OK;
  if ((phases & BE_RUN_ATTENTION) && info->grid_items > 0) {
    switch (info->dtype) {
      case BE_F32: rc = launch_attn<float>(info, a, st); break;
      case BE_F16: rc = launch_attn<f16_t>(info, a, st); break;
      case BE_BF16: rc = launch_attn<bf16_t>(info, a, st); break;
      default: return fail(BE_ERR_INVALID, "dtype %d", info->dtype);
    }
    if (rc) return rc;
  }
  if (!(phases & BE_RUN_MERGE)) return rc;
  MergeArgs m;
  m.part_o = a.part_o; m.part_lse = a.part_lse;
  m.merge_rows = plan + info->off_merge_rows;
  m.out = out; m.o_sn = o_sn; m.o_sh = o_sh; m.out_lse = lse; m.hq = info->num_qo_heads;
  for (int pass = 0; pass < 2; ++pass) {
    // pass 0: split-K merge (separate-merge plans); pass 1: queries without keys
    const int count = pass == 0 ? (info->fused_merge ? 0 : info->grid_merge) : info->grid_zero;
    if (count == 0) continue;
    m.live = info->static_layout ? plan + (pass == 0 ? kHdrMerge : kHdrZero) : nullptr;
    m.merge_q = plan + (pass == 0 ? info->off_merge_q : info->off_zero_q);
    m.merge_ptr = plan + (pass == 0 ? info->off_merge_ptr : info->off_zero_ptr);
    switch (info->dtype) {
      case BE_F32: rc = launch_merge<float>(info, m, count, st); break;
      case BE_F16: rc = launch_merge<f16_t>(info, m, count, st); break;
      case BE_BF16: rc = launch_merge<bf16_t>(info, m, count, st); break;
    }
    if (rc) return rc;
  }
  return rc;
}

}  // namespace be

extern "C" {

int be_attn_plan(const be_level* levels, int num_levels, int num_queries, int num_qo_heads,
                 int num_kv_heads, int head_dim, int page_size, int num_pages, int dtype, int flags,
                 int num_cus, const be_plan_caps* caps, int32_t* host_plan, int64_t host_plan_capacity,
                 be_attn_plan_info* info) {
  return be::attn_plan(levels, num_levels, num_queries, num_qo_heads, num_kv_heads, head_dim, page_size,
                       num_pages, dtype, flags, num_cus, caps, host_plan, host_plan_capacity, info);
}

int be_attn_run(const be_attn_plan_info* info, const int32_t* dev_plan, void* partials, const void* q,
                int64_t q_stride_n, int64_t q_stride_h, const void* kv_layer, void* out, int64_t o_stride_n,
                int64_t o_stride_h, float* lse, float sm_scale, int phases, void* stream) {
  return be::attn_run(info, dev_plan, partials, q, q_stride_n, q_stride_h, kv_layer, out, o_stride_n,
                      o_stride_h, lse, sm_scale, phases, stream);
}

int be_merge_states(const float* o_a, const float* lse_a, const float* o_b, const float* lse_b, float* o_out,
                    float* lse_out, int n, int heads, int head_dim, void* stream) {
  BE_REQUIRE(o_a && lse_a && o_b && lse_b && o_out && lse_out, "null pointer");
  BE_REQUIRE(n >= 0 && heads > 0 && head_dim > 0, "bad shape");
  const int64_t rows = (int64_t)n * heads;
  const int64_t total = rows * head_dim;
  if (total == 0) return BE_OK;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  be::merge2_kernel<<<(unsigned)((rows + 3) / 4), 256, 0, st>>>(o_a, lse_a, o_b, lse_b, o_out, lse_out,
                                                              (int)rows, head_dim);
  BE_HIP_CHECK(hipGetLastError());
  return BE_OK;
}

}  // extern "C"

// Persistent streaming decode attention for gfx950 (bf16 / fp16 KV, head_dim 128).
//
// The same quantities as the tile kernel in attention.hip — softmax(s q K^T) V
// of every query over each of its cascade groups, merged by log-sum-exp — as
// FlashInfer's MultiLevelCascadeAttentionWrapper computes them for the
// reference (models/modeling_llama.py:321-367, 732-755), but scheduled for an
// HBM-bound decode step on MI355X:
//
//  * One workgroup (8 waves) per CU.  The planner cuts the work — (query tile
//    of <= 64 rows) x (KV head) x (64-token tiles) — into one contiguous run per
//    workgroup with equal cost, splitting work items at tile boundaries where a
//    run ends.  A piece of a work item inside one run is a segment.  Groups of
//    at most 128 tokens and 4 queries skip this kernel: the tail-and-merge
//    kernel attends them per (query, KV head).
//  * Two loops.  Workgroups of at least kRegsMinTiles tiles move K, V and Q
//    rows global -> registers -> LDS: two register sets keep the loads of
//    tiles n + 1 and n + 2 in flight (across segment boundaries) while tile n
//    is computed from one of 2 LDS stages of {K 16 KB, V 16 KB, Q slot 16 KB};
//    iteration n computes n, stores tile n + 1 into the other stage, loads
//    tile n + 3.  (Direct global->LDS loads of the same 256-byte rows streamed
//    at 4.8 TB/s on MI355X, 6.2 TB/s through registers.)  Shorter workgroups
//    use direct global->LDS loads (global_load_lds_dwordx4, explicit vmcnt
//    waits, 3 stages, tile n + 2 issued in iteration n): they reach their
//    first tile sooner.  The page size is a multiple of 16, so each wave's 8
//    rows of a tile lie in one page whose id is a scalar load, issued an
//    iteration early.
//  * K, V and Q rows are 256-byte rows whose 16-byte chunks sit XOR-swizzled by
//    row (the swizzle is applied by choosing each lane's global address, since
//    a direct load writes lane l's 16 bytes at LDS base + 16 l).
//  * S^T = K Q^T with v_mfma_f32_16x16x32 (A = K rows, B = Q from registers);
//    the C layout of a 16-token S^T tile is the B operand (P^T) of
//    v_mfma_f32_16x16x16 for O^T = V^T P^T.  Its A operand (4 consecutive
//    tokens of one head_dim column) is read from the row-major V tile with
//    ds_read_b64_tr_b16: in each 16-lane group, lane r supplies the address of
//    V[t0 + r/4][d0 + 4 (r%4) .. +3] and receives V[t0 + j][d0 + r], j = 0..3.
//  * Waves split a segment's rows (16-row MFMA tiles), tokens and head_dim by
//    the segment's row count (modes below).  Long groups of more than 64 rows
//    (many beams x GQA group) get 128-row segments whose waves hold 32 rows
//    each, so a tile is read once per 128 rows; online softmax in the log2
//    domain, fp32 accumulation, natural-log lse at the boundary.
//  * A (query, KV head) covered by one segment is written as the final
//    output; otherwise each segment writes a partial (o, lse) slot and a
//    merge record combines the slots of the (query, KV head).  A slot holds
//    the normalised o in the KV's 16-bit type (the type FlashInfer's cascade
//    merges its per-level outputs in) and the lse in fp32: half the bytes of
//    fp32 slots, which the launch writes and reads back once each.  Outputs
//    are written with non-temporal stores and slots written through to the
//    device's point of coherence: nothing in the launch reads them back, and
//    the end-of-kernel write-back before the merge kernel then has little
//    left to do (the gap between the two kernels halved on MI355X).

#include <math.h>

#include <algorithm>
#include <vector>

#include "attention.h"
#include "stream_device.h"

namespace be {

namespace stream {

constexpr int kDmaStages = 3;                 // LDS stages of the direct-load loop
constexpr int kRegStages = 2;                 // LDS stages of the register-staged loop
constexpr int kRegsMinTiles = 8;              // launches whose largest run has this many tiles stage through registers
constexpr int kSegRows = 64;                  // rows per segment: 4 waves x 16
constexpr int kMaxSegs = 224;                 // segments per workgroup (LDS table)
constexpr int kKvBytes = kTok * kD * 2;       // one K (or V) tile: 16 KB
constexpr int kQBytes = kSegRows * kD * 2;    // one Q slot: 16 KB
constexpr int kStageBytes = 2 * kKvBytes + kQBytes;
constexpr int kLdsStages = kRegStages * kStageBytes;   // the smaller of the two loops' stage buffers
constexpr int kClassGeneric = 1;              // workgroup-table class: per-segment mode (else the mode 0 or 2)
constexpr int kClassWide = 5;                 // workgroup-table class of the wide roles (32 rows per wave)
constexpr int kClassWide256 = 6;              // ... of the 256-row wide roles (32 rows x all tokens per wave)
constexpr int kClassWide256Dma = 7;           // ... the same through the direct-load loop (BE_PLAN_NO_REGS)
constexpr int kNoCausalS = 0x3fffffff;        // segment causal base of a segment without the mask
constexpr int kWaves = 8;                     // 2 per SIMD; each head_dim half gets 4
constexpr int kThreads = 64 * kWaves;
constexpr int kSegCost = 4;                   // planner cost of a segment start, in quarter tiles
constexpr int kQuarterTiles = 4;              // single-row-tile segments this long split tokens 4 ways
constexpr int kTailTokens = 128;              // groups this short with few queries go to the tail pass
constexpr int kTailQueries = 4;
constexpr int kTailChunks = 64;               // 16-token tail chunks per query (one per lane)
constexpr int kRecWords = 8;                  // int32 words per merge record (and per tail item)
constexpr int kTailRole = 8;                  // workgroup-table class of a workgroup that runs tail items
constexpr int kTailUnit = 1;                  // planner cost of one tail chunk of one KV head (a tile is 4)
constexpr int kTailRoleChunks = 2;            // tail chunks per query up to which the tail role is the default
constexpr int kItemChunks = 4;                // tail chunks per tail item (tail role and tail queue)
constexpr int kWideRows = 128;               // rows per segment of a long group's wide-128 tasks
constexpr int kWideMinTiles = 8;              // 128-row tasks for groups of at least this many tiles
constexpr int kWideMinRun = 64;               // ... when the launch has this many 64-row tiles per workgroup
constexpr int kWideTileCost = 6;              // planner cost of a 128-row tile (a 64-row tile is 4)
constexpr int kWide256Rows = 256;             // rows per segment of the 256-row wide tasks
// planner cost of a 256-row tile.  Such a tile's step is bound by MFMA and
// LDS, not by its bytes: beside 64-row and shorter segments in one launch
// (config 5's long suffixes) it runs at about 1.5x, not 2.5x, a 16-row tile's
// time on MI355X, and the 2.5x weight left those workgroups finishing 80 us
// after the wide ones (286.8 -> 240.7 us per launch, 238-244 over four suffix
// seeds, with 6)
constexpr int kWide256TileCost = 6;
// planner cost of a 256-row segment start (a second segment in a workgroup:
// its epilogue, the next segment's Q rows, the pipeline across the switch).
// Measured on MI355X at config 5: such workgroups ended 9 us (about 3.4
// 256-row tiles) after one-segment ones at the cost of 4; with 24, 1.5-2%
// shorter launches over four suffix seeds (20 and 28 within 0.5%)
constexpr int kWide256SegCost = 24;

struct StreamSeg {
  int32_t q_begin;     // first query
  int32_t q_count;     // queries; rows = q_count * group <= 64
  int32_t page_begin;  // first entry of the plan's page list for the group
  int32_t tok_begin;   // first group token of the segment (a multiple of 64)
  int32_t tok_count;   // tokens, > 0
  int32_t head;        // KV head
  int32_t out_slot;    // first partial slot (one per query), or -1: final output
  int32_t n_tiles;     // ceil(tok_count / 64)
};
static_assert(sizeof(StreamSeg) == 32, "segment record is 8 int32 words");

struct StreamArgs {
  const void* q;
  int64_t q_sn, q_sh;
  const void* kv;
  void* out;
  int64_t o_sn, o_sh;
  float* out_lse;
  void* part_o;       // [slots, g, D] in the KV's 16-bit type
  float* part_lse;    // [slots, g]
  const int4* wg;     // per workgroup: first segment (item), segments (items), tiles, class
  const StreamSeg* segs;
  const int32_t* seg_causal;   // per segment: tokens its first query sees (causal), or null
  const int32_t* titems;   // tail items [n][8]: query, KV head, first tail chunk, chunks, slot
  const int2* tails;
  const int32_t* pages;
  int page_size, page_shift, hkv, hq, g;
  float scale_log2;
};

struct TailMergeArgs {
  const void* part_o;        // [slots, g, D] in the KV's 16-bit type
  const float* part_lse;
  const int32_t* recs;       // [n][8]: query, KV head, first rec_slots entry, slots, first tail, tails, 0, 0
  const int32_t* rec_slots;
  const int2* tails;         // 16-token chunks: page id, in-page token offset | valid tokens << 16
  const int32_t* live;       // live record count (device), or null
  const void* q;
  int64_t q_sn, q_sh;
  const void* kv;
  void* out;
  int64_t o_sn, o_sh;
  float* out_lse;
  int n_recs, g, hq, hkv, page_size;
  float scale_log2;
};

// A segment record held in wave-uniform registers.
struct SegReg {
  int q_begin, q_count, page_begin, tok_begin, tok_count, head, out_slot, n_tiles;
};
__device__ __forceinline__ SegReg seg_reg(const StreamSeg& x) {
  return SegReg{rfl(x.q_begin), rfl(x.q_count), rfl(x.page_begin), rfl(x.tok_begin),
                rfl(x.tok_count), rfl(x.head),   rfl(x.out_slot),   rfl(x.n_tiles)};
}

// The end of a wide role's 16-row tile: lane holds O^T[d = 16 mt + 4 lg + i]
// [row] of segment row `row` (< rows), normalised by l, with m in the log2
// domain; to the final output or the segment's partial slot.
template <typename T>
__device__ __forceinline__ void wide_store(const StreamArgs& a, const SegReg& sg, int row, int lg, float m, float l,
                                           const v4f (&o)[8]) {
  const int g = a.g;
  const int j = row / g, hh = row - j * g, head = sg.head * g + hh;
  const int qi = sg.q_begin + j;
  const float inv = (l > 0.f) ? 1.f / l : 0.f;
  const float lse = (l > 0.f) ? (m + log2f(l)) * 0.69314718055994531f : -INFINITY;
  const int d0 = 4 * lg;
  if (sg.out_slot < 0) {
    T* op = reinterpret_cast<T*>(a.out) + (int64_t)qi * a.o_sn + (int64_t)head * a.o_sh + d0;
#pragma unroll
    for (int mt = 0; mt < 8; ++mt)
      __builtin_nontemporal_store(pack4<T>(o[mt][0] * inv, o[mt][1] * inv, o[mt][2] * inv, o[mt][3] * inv),
                                  reinterpret_cast<v4s*>(op + mt * 16));
    if (lg == 0 && a.out_lse) __builtin_nontemporal_store(lse, a.out_lse + (int64_t)qi * a.hq + head);
  } else {
    const int64_t slot = (int64_t)(sg.out_slot + j) * g + hh;
    T* op = reinterpret_cast<T*>(a.part_o) + slot * kD + d0;
#pragma unroll
    for (int mt = 0; mt < 8; ++mt)
      store_wt(reinterpret_cast<v4s*>(op + mt * 16),
               pack4<T>(o[mt][0] * inv, o[mt][1] * inv, o[mt][2] * inv, o[mt][3] * inv));
    if (lg == 0) store_wt(a.part_lse + slot, lse);
  }
}

// Online softmax of one (query, KV head) over its tail chunks c = first,
// first + stride, ... < nt (16 tokens of one page each; ent: lane k holds
// chunk k's page id and in-page offset | valid << 16).  K and V rows go from
// global memory through registers (NB chunks in flight, 32 VGPRs each) into
// the wave's 8 KB LDS area and the streaming tile step, rows = the g query
// heads of the KV head.  A token in two groups counts twice, as two merged
// groups would count it.
template <typename T, int NB = 2>
__device__ __forceinline__ void tail_chunks(const void* q, int64_t q_sn, int64_t q_sh, const void* kv, int ps, int hkv,
                                            int g, int qi, int h, int2 ent, int nt, int first, int stride,
                                            unsigned char* area, float scale, float& m_run, float& l_run,
                                            v4f (&o_acc)[8]) {
  typedef int v4i __attribute__((ext_vector_type(4)));
  const int lane = threadIdx.x & 63, lg = lane >> 4, lc = lane & 15;
  unsigned char* kt = area;
  unsigned char* vt = area + 4096;
  const T* kvp = reinterpret_cast<const T*>(kv);
  const int64_t plane = (int64_t)ps * hkv * kD;
  const T* qp = reinterpret_cast<const T*>(q) + (int64_t)qi * q_sn + (int64_t)(h * g + min(lc, g - 1)) * q_sh;
  v8s qf[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) qf[ks] = *reinterpret_cast<const v8s*>(qp + 8 * (4 * ks + lg));
  uint32_t koff[4], voff8[8];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) koff[ks] = lc * 256 + ((((ks << 2) | lg) ^ lc) << 4);
  {
    const int tl = 4 * lg + (lc >> 2), b1 = (lc >> 1) & 1, b0 = lc & 1;
#pragma unroll
    for (int mt = 0; mt < 8; ++mt) voff8[mt] = (uint32_t)(tl * 256 + ((((2 * mt) | b1) ^ tl) << 4) + (b0 << 3));
  }
  // rows 4 i + lg of chunk c, 16-byte column slot lc holding global column lc ^ row,
  // into register buffer b
  v4i kr[NB][4], vr[NB][4];
  auto load = [&](int c, int b) {
    const int page = __builtin_amdgcn_readlane(ent.x, c);
    const int ov = __builtin_amdgcn_readlane(ent.y, c);
    const int off = ov & 0xffff, valid = ov >> 16;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 4 * i + lg;
      const int tok = off + min(r, valid - 1);
      const T* src = kvp + (((int64_t)page * 2 * ps + tok) * hkv + h) * kD + ((lc ^ r) << 3);
      kr[b][i] = *reinterpret_cast<const v4i*>(src);
      vr[b][i] = *reinterpret_cast<const v4i*>(src + plane);
    }
  };
  // chunk c from buffer b to LDS, chunk c + NB stride into buffer b, then compute c
  auto step = [&](int c, int b) {
    const int valid = __builtin_amdgcn_readlane(ent.y, c) >> 16;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 4 * i + lg;
      *reinterpret_cast<v4i*>(kt + r * 256 + lc * 16) = kr[b][i];
      *reinterpret_cast<v4i*>(vt + r * 256 + lc * 16) = vr[b][i];
    }
    if (c + NB * stride < nt) load(c + NB * stride, b);
    tile_compute<T, 1, 8>(kt, vt, qf, koff, voff8, 0, valid, lg, scale, m_run, l_run, o_acc);
  };
#pragma unroll
  for (int b = 0; b < NB; ++b)
    if (first + b * stride < nt) load(first + b * stride, b);
  for (int c = first; c < nt; c += NB * stride) {
#pragma unroll
    for (int b = 0; b < NB; ++b)
      if (c + b * stride < nt) step(c + b * stride, b);
  }
}

// The loop of one workgroup over its segments' tiles, K, V and Q rows by
// direct global->LDS loads (the planner's choice for workgroups of few tiles,
// whose time is mostly the pipeline's fill and drain, and for the wide
// roles).  Three LDS stages; iteration n waits for tile n, issues the loads
// of tile n + 2 and computes tile n.  FM as for stream_body_regs, or
// kClassWide: the wide roles (32 rows per wave, segments of up to 128 rows);
// kClassWide256: the same with segments of up to 256 rows, every wave over
// all 64 tokens of a tile.
template <typename T, int FM>
__device__ __forceinline__ void stream_body_dma(const StreamArgs& a, unsigned char* st_lds, StreamSeg* seg_lds,
                                                const int* vis_lds, float* ml_lds, int n_segs, int n_tiles) {
  const int tid = threadIdx.x;
  const int w = rfl(tid >> 6);                        // wave index (uniform)
  const int lane = tid & 63, lg = lane >> 4, lc = lane & 15;
  const int ps = a.page_size, g = a.g, hkv = a.hkv;
  const int pshift = a.page_shift;
  auto page_of = [&](int tok) { return pshift >= 0 ? (tok >> pshift) : (tok / ps); };
  const T* kv = reinterpret_cast<const T*>(a.kv);
  const int64_t plane = (int64_t)ps * hkv * kD;      // K plane -> V plane of a page (elements)
  const uint32_t st0 = lds_addr(st_lds);
  const float scale = a.scale_log2;

  // per-lane LDS offsets (bytes) of the MFMA operand reads, within a 16-token
  // sub-tile: K / Q rows, and V^T columns of all 8 head_dim tiles, of this
  // wave's half (waves 4..7 take the upper half) and of head_dim tile w
  uint32_t koff[4], voff8[8], voff4[4], voff1[1];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) koff[ks] = lc * 256 + ((((ks << 2) | lg) ^ lc) << 4);
  {
    const int tl = 4 * lg + (lc >> 2), b1 = (lc >> 1) & 1, b0 = lc & 1;
    auto vcol = [&](int mt) { return (uint32_t)(tl * 256 + ((((2 * mt) | b1) ^ tl) << 4) + (b0 << 3)); };
#pragma unroll
    for (int mt = 0; mt < 8; ++mt) voff8[mt] = vcol(mt);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) voff4[mt] = vcol(4 * (w >> 2) + mt);
    voff1[0] = vcol(w);
  }
  // this wave loads rows 8w..8w+7 of every tile (two 1 KB loads of 4 rows for
  // K and for V).  The page size is a multiple of 16 and tiles start at a
  // multiple of 64 tokens, so the 8 rows lie in one page: one page id (a
  // scalar load) and per-lane row offsets from the wave's first row.
  uint32_t doff[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int r = 4 * i + lg;
    doff[i] = (uint32_t)(((int64_t)r * hkv * kD + ((lc ^ (8 * (w & 1) + r)) << 3)) * 2);
  }

  // cursors: segment index, tile of the segment and the segment's record, for
  // the K/V/Q loads and for the compute
  int l_s = 0, l_t = 0, c_s = 0, c_t = 0;
  SegReg l_sg = seg_reg(seg_lds[0]), c_sg = l_sg;
  auto advance = [&](int& si, int& ti, SegReg& sg) {
    if (++ti == sg.n_tiles) {
      ti = 0;
      if (++si < n_segs) sg = seg_reg(seg_lds[si]);
    }
  };
  // the page id of this wave's rows of the next tile to load (load cursor);
  // read before the wait of an iteration so that its latency hides there
  auto page_id = [&]() -> int {
    const int valid = min(kTok, l_sg.tok_count - l_t * kTok);
    const int t8 = l_sg.tok_begin + l_t * kTok + min(8 * w, valid - 1);
    typedef const __attribute__((address_space(4))) int32_t* const_i32_t;   // scalar (constant) loads
    return ((const_i32_t)(uintptr_t)a.pages)[rfl(l_sg.page_begin + page_of(t8))];
  };

  // Loads of the next tile (load cursor) into stage st: the Q rows now when the
  // tile starts a segment; the K/V rows are prepared here and issued by dma(j).
  bool kv_pending = false;
  uint64_t kv_kbase = 0, kv_vbase = 0;
  uint32_t kv_off[2] = {0, 0};
  uint32_t kv_lds = 0;
  auto prep_tile = [&](int st, int page) -> int {
    const SegReg& sg = l_sg;
    const uint32_t stage = st0 + (uint32_t)(st * kStageBytes);
    const int valid = min(kTok, sg.tok_count - l_t * kTok);
    const int r0 = min(8 * w, valid - 1);             // rows past the end re-read the last token
    const int t8 = sg.tok_begin + l_t * kTok + r0;
    const int s0 = t8 - page_of(t8) * ps;
    kv_pending = true;
    kv_lds = stage + (2 * w) * 1024;
    kv_kbase = reinterpret_cast<uint64_t>(kv) + (uint64_t)(((((int64_t)page * 2) * ps + s0) * hkv + sg.head) * kD * 2);
    kv_vbase = kv_kbase + (uint64_t)(plane * 2);
    if (8 * w + 8 <= valid) {
      kv_off[0] = doff[0];
      kv_off[1] = doff[1];
    } else {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int r = 4 * i + lg;
        const int rel = min(8 * w + r, valid - 1) - r0;
        kv_off[i] = (uint32_t)(((int64_t)rel * hkv * kD + ((lc ^ (8 * (w & 1) + r)) << 3)) * 2);
      }
    }
    int ops = 4;                                      // K/V loads per wave per tile
    if (FM != kClassWide && FM != kClassWide256 && l_t == 0) {   // wide roles: Q rows go to registers
      const int R = sg.q_count * g;
      const int nq = (R + 3) >> 2;                    // 1 KB loads of 4 rows
      for (int k = w; k < nq; k += kWaves) {
        const int r = 4 * k + lg;
        const int rc = min(r, R - 1);
        const int j = rc / g, hh = rc - j * g;
        const T* src = reinterpret_cast<const T*>(a.q) + (int64_t)(sg.q_begin + j) * a.q_sn +
                       (int64_t)(sg.head * g + hh) * a.q_sh + ((lc ^ (r & 15)) << 3);
        dma16(src, stage + 2 * kKvBytes + k * 1024);
        ++ops;
      }
    }
    advance(l_s, l_t, l_sg);
    return ops;
  };
  // the four loads of the prepared tile: K rows 0..3, V rows 0..3, K rows 4..7, V rows 4..7
  auto dma_all = [&]() {
    if (!kv_pending) return;
    dma16_sv(kv_kbase, kv_off[0], kv_lds);
    dma16_sv(kv_vbase, kv_off[0], kv_lds + kKvBytes);
    dma16_sv(kv_kbase, kv_off[1], kv_lds + 1024);
    dma16_sv(kv_vbase, kv_off[1], kv_lds + kKvBytes + 1024);
  };

  // ---- prologue.  Iteration i issues the loads of tile i + 2, then computes
  // tile i (its epilogue stores come last).  Waiting until only the previous
  // iteration's operations are outstanding therefore completes everything
  // issued two iterations back: tile i's K/V/Q.
  prep_tile(0, page_id());
  dma_all();
  int ops_prev = 0;                  // operations issued by the previous iteration
  if (n_tiles > 1) {
    ops_prev = prep_tile(1, page_id());
    dma_all();
  }
  kv_pending = false;

  float m_run = -INFINITY, l_run = 0.f;
  v4f o_acc[8];
  v8s qf[4];
  float m2[2] = {-INFINITY, -INFINITY}, l2[2] = {0.f, 0.f};   // wide roles
  v4f o2[2][8];
  v4f lw[2];                                                    // 256-row wide roles: row sums
  v8s qf2[2][4];
  int st_c = 0, st_l = 2;            // stages of the computed and the next loaded tile

  for (int n = 0; n < n_tiles; ++n) {
    const int page = (n + 2 < n_tiles) ? page_id() : 0;
    wait_vmcnt(rfl(ops_prev));
    lds_fence();
    int ops = 0;
    if (n + 2 < n_tiles) {
      ops += prep_tile(st_l, page);
      dma_all();
    }
    kv_pending = false;
    st_l = st_l == kDmaStages - 1 ? 0 : st_l + 1;

    // ---- compute tile n.  Wave roles by the segment's row tiles (NT):
    //   NT >= 3: row tile w & 3, token half w >> 2, all head_dim        (mode 0)
    //   NT == 2: row tile w & 1, token half (w >> 1) & 1, head_dim half  (mode 1)
    //   NT == 1, segment of >= kQuarterTiles tiles: token quarter w & 3,
    //            head_dim half w >> 2                                     (mode 2)
    //   NT == 1, shorter: all 64 tokens, head_dim tile w                  (mode 3)
    // Where tokens are split, the ts == 0 wave of each (row tile, head_dim
    // part) collects the others at the end of the segment; mode 3 recomputes
    // the scores in every wave instead, which costs less than that exchange
    // when the segment is short.
    if constexpr (FM != kClassWide && FM != kClassWide256) {
    const SegReg& sg = c_sg;
    const int R = sg.q_count * g;
    const int NT = (R + 15) >> 4;
    const int mode = FM >= 0 ? FM : NT >= 3 ? 0 : NT == 2 ? 1 : sg.n_tiles >= kQuarterTiles ? 2 : 3;
    const int rt = mode == 0 ? (w & 3) : mode == 1 ? (w & 1) : 0;
    const int ts = mode == 0 ? (w >> 2) : mode == 1 ? ((w >> 1) & 1) : mode == 2 ? (w & 3) : 0;
    const int sub0 = mode == 2 ? ts : 2 * ts;
    const bool act = 16 * rt < R;
    const bool last = c_t == sg.n_tiles - 1;
    unsigned char* stage = st_lds + st_c * kStageBytes;
    if (c_t == 0) {
      m_run = -INFINITY;
      l_run = 0.f;
#pragma unroll
      for (int mt = 0; mt < 8; ++mt) o_acc[mt] = v4f{0.f, 0.f, 0.f, 0.f};
      if (act) {
        const unsigned char* qs = stage + 2 * kKvBytes + rt * 4096;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) qf[ks] = *reinterpret_cast<const v8s*>(qs + koff[ks]);
      }
    }
    if (act) {
      const int valid = min(kTok, sg.tok_count - c_t * kTok);
      const int vr = row_limit(valid, vis_lds[c_s], 16 * rt + lc, g, sg.tok_begin + c_t * kTok);
      const unsigned char* kt = stage + sub0 * 4096;
      const unsigned char* vt = stage + kKvBytes + sub0 * 4096;
      if (mode == 0)
        tile_compute<T, 2, 8>(kt, vt, qf, koff, voff8, sub0 * 16, vr, lg, scale, m_run, l_run, o_acc);
      else if (mode == 1)
        tile_compute<T, 2, 4>(kt, vt, qf, koff, voff4, sub0 * 16, vr, lg, scale, m_run, l_run, o_acc);
      else if (mode == 2)
        tile_compute<T, 1, 4>(kt, vt, qf, koff, voff4, sub0 * 16, vr, lg, scale, m_run, l_run, o_acc);
      else
        tile_compute<T, 4, 1>(kt, vt, qf, koff, voff1, 0, vr, lg, scale, m_run, l_run, o_acc);
    }

    if (last) {
      float l = l_run;
      l = rows4_sum(l);
      const int nmt = mode == 0 ? 8 : mode == 3 ? 1 : 4;
      const int mt0 = mode == 0 ? 0 : mode == 3 ? w : 4 * (w >> 2);
      // token-split waves hand their state to the ts == 0 wave of their (row
      // tile, head_dim part): o through this stage's K/V area (no loads target
      // it until the next iteration's barrier; at most 32 KB), m and l through
      // ml_lds
      const int kslot = nmt * 1024;
      if (mode != 3) lds_sync();
      if (ts > 0 && act) {
        unsigned char* slot = stage + (mode == 0 ? w - 4 : w) * kslot;
#pragma unroll
        for (int mt = 0; mt < 8; ++mt)
          if (mt < nmt) *reinterpret_cast<v4f*>(slot + (mt * 64 + lane) * 16) = o_acc[mt];
        ml_lds[w * 128 + lane] = m_run;
        ml_lds[w * 128 + 64 + lane] = l;
      }
      if (mode != 3) lds_sync();
      if (ts == 0 && act) {
        const int np = mode == 2 ? 4 : mode == 3 ? 1 : 2;   // waves sharing the (row tile, head_dim part)
        for (int p = 1; p < np; ++p) {
          const int pw = mode == 0 ? w + 4 : mode == 1 ? w + 2 : w + p;   // partner wave
          const unsigned char* slot = stage + (mode == 0 ? pw - 4 : pw) * kslot;
          const float mb = ml_lds[pw * 128 + lane];
          const float lb = ml_lds[pw * 128 + 64 + lane];
          const float M = fmaxf(m_run, mb);
          const float ca = (M == -INFINITY) ? 0.f : exp2f(m_run - M);
          const float cb = (M == -INFINITY) ? 0.f : exp2f(mb - M);
          l = l * ca + lb * cb;
          m_run = M;
#pragma unroll
          for (int mt = 0; mt < 8; ++mt)
            if (mt < nmt)
              o_acc[mt] = o_acc[mt] * ca + *reinterpret_cast<const v4f*>(slot + (mt * 64 + lane) * 16) * cb;
        }
        // lane holds O^T[d = 16 (mt0 + mt) + 4 lg + i][row = 16 rt + lc]
        const int row = 16 * rt + lc;
        if (row < R) {
          const int j = row / g, hh = row - j * g, head = sg.head * g + hh;
          const int qi = sg.q_begin + j;
          const float inv = (l > 0.f) ? 1.f / l : 0.f;
          const float lse = (l > 0.f) ? (m_run + log2f(l)) * 0.69314718055994531f : -INFINITY;
          const int d0 = 16 * mt0 + 4 * lg;
          if (sg.out_slot < 0) {
            T* op = reinterpret_cast<T*>(a.out) + (int64_t)qi * a.o_sn + (int64_t)head * a.o_sh + d0;
#pragma unroll
            for (int mt = 0; mt < 8; ++mt)
              if (mt < nmt)
                __builtin_nontemporal_store(
                    pack4<T>(o_acc[mt][0] * inv, o_acc[mt][1] * inv, o_acc[mt][2] * inv, o_acc[mt][3] * inv),
                    reinterpret_cast<v4s*>(op + mt * 16));
            if (mt0 == 0 && lg == 0 && a.out_lse) __builtin_nontemporal_store(lse, a.out_lse + (int64_t)qi * a.hq + head);
          } else {
            const int64_t slot = (int64_t)(sg.out_slot + j) * g + hh;
            T* op = reinterpret_cast<T*>(a.part_o) + slot * kD + d0;
#pragma unroll
            for (int mt = 0; mt < 8; ++mt)
              if (mt < nmt)
                store_wt(reinterpret_cast<v4s*>(op + mt * 16),
                         pack4<T>(o_acc[mt][0] * inv, o_acc[mt][1] * inv, o_acc[mt][2] * inv, o_acc[mt][3] * inv));
            if (mt0 == 0 && lg == 0) store_wt(a.part_lse + slot, lse);
          }
        }
        ops += nmt;                                      // store instructions (lse not counted)
      }
    }
    } else {
    // ---- wide roles (every segment of the workgroup).  kClassWide (up to 128
    // rows): wave w takes rows 32 (w & 3) .. +31 as two 16-row MFMA tiles
    // sharing each K / V^T fragment read, and tokens 32 (w >> 2) .. +31 of the
    // tile; the w < 4 wave of each row group collects its partner's (m, l, o)
    // at the end of the segment, one row tile at a time through this stage.
    // kClassWide256 (up to 256 rows): wave w takes rows 32 w .. +31 and every
    // token of the tile (two 32-token steps), so a tile is read once per 256
    // rows and no wave hands over.  The segment's Q rows go global ->
    // registers on its first tile (more than the stage's Q slot holds).
    constexpr int TP = FM == kClassWide256 ? 1 : 2;   // token parts
    constexpr int RG = kWaves / TP;                   // 32-row groups
    constexpr int NSUB = 4 / TP;                      // 16-token sub-tiles per part
    const int rg = w % RG, tp = w / RG;
    const SegReg& sg = c_sg;
    const int R = sg.q_count * g;
    const bool act = 32 * rg < R;
    const bool last = c_t == sg.n_tiles - 1;
    unsigned char* stage = st_lds + st_c * kStageBytes;
    if (c_t == 0) {
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        m2[r] = -INFINITY;
        l2[r] = 0.f;
        lw[r] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int mt = 0; mt < 8; ++mt) o2[r][mt] = v4f{0.f, 0.f, 0.f, 0.f};
      }
      if (act) {
        {
          // rows past the segment's last re-read it (their results are never stored)
#pragma unroll
          for (int r = 0; r < 2; ++r) {
            const int row = min(32 * rg + 16 * r + lc, R - 1);
            const int j = row / g, hh = row - j * g;
            const T* src = reinterpret_cast<const T*>(a.q) + (int64_t)(sg.q_begin + j) * a.q_sn +
                           (int64_t)(sg.head * g + hh) * a.q_sh;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) qf2[r][ks] = *reinterpret_cast<const v8s*>(src + 8 * (4 * ks + lg));
          }
        }
      }
    }
    if (act) {
      const int valid = min(kTok, sg.tok_count - c_t * kTok);
      if constexpr (TP == 1) {
        tile_compute_w64<T>(stage, stage + kKvBytes, qf2, koff, voff8, valid, lg, scale, m2, lw, o2);
      } else {
        const int sub0 = tp * NSUB;
        tile_compute_w<T, NSUB>(stage + sub0 * 4096, stage + kKvBytes + sub0 * 4096, qf2, koff, voff8, sub0 * 16,
                                valid, lg, scale, m2, l2, o2);
      }
    }
    if (last) {
      float l[2];
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        // (256-row roles: every lane's l is the whole row's, from the MFMA pipe)
        l[r] = TP == 1 ? lw[r][0] : rows4_sum(l2[r]);
      }
      // (TP - 1) * RG = 4 waves hand over 8 KB each per row tile (32 KB of the stage's 48)
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        lds_sync();
        if (tp > 0 && act) {
          unsigned char* slot = stage + ((tp - 1) * RG + rg) * 8192;
#pragma unroll
          for (int mt = 0; mt < 8; ++mt) *reinterpret_cast<v4f*>(slot + (mt * 64 + lane) * 16) = o2[r][mt];
          ml_lds[w * 128 + lane] = m2[r];
          ml_lds[w * 128 + 64 + lane] = l[r];
        }
        lds_sync();
        if (tp == 0 && act) {
#pragma unroll
          for (int p = 1; p < TP; ++p) {
            const int pw = p * RG + rg;
            const unsigned char* slot = stage + ((p - 1) * RG + rg) * 8192;
            const float mb = ml_lds[pw * 128 + lane];
            const float lb = ml_lds[pw * 128 + 64 + lane];
            const float M = fmaxf(m2[r], mb);
            const float ca = (M == -INFINITY) ? 0.f : exp2f(m2[r] - M);
            const float cb = (M == -INFINITY) ? 0.f : exp2f(mb - M);
            l[r] = l[r] * ca + lb * cb;
            m2[r] = M;
#pragma unroll
            for (int mt = 0; mt < 8; ++mt)
              o2[r][mt] = o2[r][mt] * ca + *reinterpret_cast<const v4f*>(slot + (mt * 64 + lane) * 16) * cb;
          }
        }
      }
      if (tp == 0 && act) {
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          const int row = 32 * rg + 16 * r + lc;
          if (row < R) wide_store<T>(a, sg, row, lg, m2[r], l[r], o2[r]);
        }
        // row tile 2 rg always has a stored row (32 rg < R): its 8 stores are
        // certain; the second tile's and the lse stores are not counted, which
        // only makes the next wait stricter
        ops += 8;
      }
    }
    }
    ops_prev = ops;
    st_c = st_c == kDmaStages - 1 ? 0 : st_c + 1;
    advance(c_s, c_t, c_sg);
  }
}

// The loop of one workgroup over its segments' tiles (the planner's choice
// for workgroups of at least kRegsMinTiles tiles, and for the 256-row wide
// roles).  FM >= 0: every segment of the workgroup takes wave-role mode FM
// (the planner marks such workgroups), so the per-tile mode dispatch folds
// away; FM < 0: mode per segment; FM == kClassWide256: the 256-row wide
// roles (wave w takes rows 32 w .. +31 over every token of a tile; the
// segment's Q rows go global -> registers on its first tile).  The 256-row
// step reads each 32 KB tile 8 times from LDS; beside it, direct
// global -> LDS loads slowed the step by about a third on MI355X, loads into
// registers stored by ds_write by about a tenth (the step with LDS-resident
// tiles: 2.0 us per tile alone, 2.7-2.9 with direct loads, 2.2 through
// registers).
//
// K, V and Q rows travel global memory -> registers -> LDS.  Two register
// sets hold tiles n + 1 and n + 2 in flight while tile n is computed from one
// of the two LDS stages; iteration n then stores tile n + 1 (loaded two
// iterations earlier) into the other stage, reloads its register set with
// tile n + 3 and ends on a barrier.  Even tiles use register set A, odd tiles
// set B (the loop is unrolled by two so that the sets are static).
template <typename T, int FM>
__device__ __forceinline__ void stream_body_regs(const StreamArgs& a, unsigned char* st_lds, StreamSeg* seg_lds,
                                                 const int* vis_lds, float* ml_lds, int n_segs, int n_tiles) {
  typedef int v4i __attribute__((ext_vector_type(4)));
  constexpr bool W256 = FM == kClassWide256;
  const int tid = threadIdx.x;
  const int w = rfl(tid >> 6);                        // wave index (uniform)
  const int lane = tid & 63, lg = lane >> 4, lc = lane & 15;
  const int ps = a.page_size, g = a.g, hkv = a.hkv;
  const int pshift = a.page_shift;
  auto page_of = [&](int tok) { return pshift >= 0 ? (tok >> pshift) : (tok / ps); };
  const T* kv = reinterpret_cast<const T*>(a.kv);
  const int64_t plane = (int64_t)ps * hkv * kD;      // K plane -> V plane of a page (elements)
  const float scale = a.scale_log2;

  // per-lane LDS offsets (bytes) of the MFMA operand reads, within a 16-token
  // sub-tile: K / Q rows, and V^T columns of all 8 head_dim tiles, of this
  // wave's half (waves 4..7 take the upper half) and of head_dim tile w
  uint32_t koff[4], voff8[8], voff4[4], voff1[1];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) koff[ks] = lc * 256 + ((((ks << 2) | lg) ^ lc) << 4);
  {
    const int tl = 4 * lg + (lc >> 2), b1 = (lc >> 1) & 1, b0 = lc & 1;
    auto vcol = [&](int mt) { return (uint32_t)(tl * 256 + ((((2 * mt) | b1) ^ tl) << 4) + (b0 << 3)); };
#pragma unroll
    for (int mt = 0; mt < 8; ++mt) voff8[mt] = vcol(mt);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) voff4[mt] = vcol(4 * (w >> 2) + mt);
    voff1[0] = vcol(w);
  }
  // this wave loads rows 8w..8w+7 of every tile (two 16-byte loads per lane
  // for K and for V, 4 rows each).  The page size is a multiple of 16 and
  // tiles start at a multiple of 64 tokens, so the 8 rows lie in one page: one
  // page id (a scalar load) and per-lane row offsets from the wave's first row.
  uint32_t doff[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int r = 4 * i + lg;
    doff[i] = (uint32_t)(((int64_t)r * hkv * kD + ((lc ^ (8 * (w & 1) + r)) << 3)) * 2);
  }

  // cursors: segment index, tile of the segment and the segment's record, for
  // the loads and for the compute
  int l_s = 0, l_t = 0, c_s = 0, c_t = 0;
  SegReg l_sg = seg_reg(seg_lds[0]), c_sg = l_sg;
  auto advance = [&](int& si, int& ti, SegReg& sg) {
    if (++ti == sg.n_tiles) {
      ti = 0;
      if (++si < n_segs) sg = seg_reg(seg_lds[si]);
    }
  };
  // the page id of this wave's rows of the next tile to load (load cursor);
  // read an iteration's compute ahead of its use so that its latency hides
  auto page_id = [&]() -> int {
    const int valid = min(kTok, l_sg.tok_count - l_t * kTok);
    const int t8 = l_sg.tok_begin + l_t * kTok + min(8 * w, valid - 1);
    typedef const __attribute__((address_space(4))) int32_t* const_i32_t;   // scalar (constant) loads
    return ((const_i32_t)(uintptr_t)a.pages)[rfl(l_sg.page_begin + page_of(t8))];
  };

  // One tile's rows in registers: K and V rows 8w + (0..3) and 8w + (4..7)
  // (lane (lg, lc) holds row 4 i + lg, 16-byte column slot lc, which holds the
  // global column lc ^ row), and, for the first tile of a segment, this wave's
  // 1 KB blocks k = w and w + 8 of the segment's Q rows.  Every call issues
  // the same six loads, each from one selected address — past the last tile
  // (live false), K/V rows of page 0 of KV head 0, and Q rows of query 0
  // head 0 where no Q block is due (cache hits, never stored) — so that the
  // compiler neither copies a set between paths nor counts fewer loads on one
  // of them when it places the waits before a set's stores.
  struct Regs {
    v4i k[2], v[2], q[2];
    int nq;                                          // Q blocks to store (0..2)
  };
  auto load = [&](Regs& r, bool live, int page) {
    const SegReg& sg = l_sg;
    const int valid = min(kTok, sg.tok_count - l_t * kTok);
    const int r0 = min(8 * w, valid - 1);             // rows past the end re-read the last token
    const int t8 = sg.tok_begin + l_t * kTok + r0;
    const int s0 = t8 - page_of(t8) * ps;
    const int64_t kb_off = live ? ((((int64_t)page * 2) * ps + s0) * hkv * kD + (int64_t)sg.head * kD) * 2 : 0;
    const char* kb = reinterpret_cast<const char*>(kv) + kb_off;
    uint32_t off[2] = {doff[0], doff[1]};
    if (live && 8 * w + 8 > valid) {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int rr = 4 * i + lg;
        const int rel = min(8 * w + rr, valid - 1) - r0;
        off[i] = (uint32_t)(((int64_t)rel * hkv * kD + ((lc ^ (8 * (w & 1) + rr)) << 3)) * 2);
      }
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      r.k[i] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(kb + off[i]));
      r.v[i] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(kb + off[i] + plane * 2));
    }
    r.nq = 0;
    if constexpr (!W256) {
    const int R = sg.q_count * g;
    const int nblk = (live && l_t == 0) ? (R + 3) >> 2 : 0;   // 1 KB blocks of 4 rows due with this tile
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int k = w + kWaves * j;
      const int rr = 4 * k + lg;
      const int rc = k < nblk ? min(rr, R - 1) : 0;
      const int qj = rc / g, hh = rc - qj * g;
      const int64_t qoff = k < nblk ? (int64_t)(sg.q_begin + qj) * a.q_sn + (int64_t)(sg.head * g + hh) * a.q_sh +
                                          ((lc ^ (rr & 15)) << 3)
                                    : (int64_t)(lc << 3);
      r.q[j] = *reinterpret_cast<const v4i*>(reinterpret_cast<const T*>(a.q) + qoff);
      if (k < nblk) r.nq = j + 1;
    }
    }
    if (live) advance(l_s, l_t, l_sg);
  };
  // store a tile's registers into stage st (lane l's 16 bytes at block + 16 l)
  auto store = [&](const Regs& r, int st) {
    unsigned char* stage = st_lds + st * kStageBytes;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      *reinterpret_cast<v4i*>(stage + (2 * w + i) * 1024 + lane * 16) = r.k[i];
      *reinterpret_cast<v4i*>(stage + kKvBytes + (2 * w + i) * 1024 + lane * 16) = r.v[i];
    }
    if constexpr (!W256) {
#pragma unroll
      for (int j = 0; j < 2; ++j)
        if (j < r.nq) *reinterpret_cast<v4i*>(stage + 2 * kKvBytes + (w + kWaves * j) * 1024 + lane * 16) = r.q[j];
    }
  };

  // ---- prologue: tiles 0 and 1 into A and B, tile 0 stored, tile 2 into A
  Regs ra, rb;
  load(ra, true, page_id());
  load(rb, n_tiles > 1, n_tiles > 1 ? page_id() : 0);
  store(ra, 0);
  load(ra, n_tiles > 2, n_tiles > 2 ? page_id() : 0);
  lds_sync();

  float m_run = -INFINITY, l_run = 0.f;
  v4f o_acc[8];
  v8s qf[4];
  float m2[2] = {-INFINITY, -INFINITY};               // 256-row wide roles: two 16-row tiles per wave
  v4f lw[2], o2[2][8];
  v8s qf2[2][4];

  // iteration n: compute n, store tile n + 1 (set nx), reload nx with tile n + 3
  auto iteration = [&](int n, Regs& nx) {
    const int page = (n + 3 < n_tiles) ? page_id() : 0;

    if constexpr (W256) {
      const SegReg& sg = c_sg;
      const int R = sg.q_count * g;
      const bool act = 32 * w < R;
      const unsigned char* stage = st_lds + (n & 1) * kStageBytes;
      if (c_t == 0) {
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          m2[r] = -INFINITY;
          lw[r] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int mt = 0; mt < 8; ++mt) o2[r][mt] = v4f{0.f, 0.f, 0.f, 0.f};
        }
        if (act) {
          // rows past the segment's last re-read it (their results are never stored)
#pragma unroll
          for (int r = 0; r < 2; ++r) {
            const int row = min(32 * w + 16 * r + lc, R - 1);
            const int j = row / g, hh = row - j * g;
            const T* src = reinterpret_cast<const T*>(a.q) + (int64_t)(sg.q_begin + j) * a.q_sn +
                           (int64_t)(sg.head * g + hh) * a.q_sh;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) qf2[r][ks] = *reinterpret_cast<const v8s*>(src + 8 * (4 * ks + lg));
          }
        }
      }
      if (act) {
        const int valid = min(kTok, sg.tok_count - c_t * kTok);
        tile_compute_w64<T>(stage, stage + kKvBytes, qf2, koff, voff8, valid, lg, scale, m2, lw, o2);
        if (c_t == sg.n_tiles - 1) {
          // every lane's l is the whole row's (row sums from the MFMA pipe)
#pragma unroll
          for (int r = 0; r < 2; ++r) {
            const int row = 32 * w + 16 * r + lc;
            if (row < R) wide_store<T>(a, sg, row, lg, m2[r], lw[r][0], o2[r]);
          }
        }
      }
    } else {

    // ---- compute tile n.  Wave roles by the segment's row tiles (NT):
    //   NT >= 3: row tile w & 3, token half w >> 2, all head_dim        (mode 0)
    //   NT == 2: row tile w & 1, token half (w >> 1) & 1, head_dim half  (mode 1)
    //   NT == 1, segment of >= kQuarterTiles tiles: token quarter w & 3,
    //            head_dim half w >> 2                                     (mode 2)
    //   NT == 1, shorter: all 64 tokens, head_dim tile w                  (mode 3)
    // Where tokens are split, the ts == 0 wave of each (row tile, head_dim
    // part) collects the others at the end of the segment; mode 3 recomputes
    // the scores in every wave instead, which costs less than that exchange
    // when the segment is short.
    const SegReg& sg = c_sg;
    const int R = sg.q_count * g;
    const int NT = (R + 15) >> 4;
    const int mode = FM >= 0 ? FM : NT >= 3 ? 0 : NT == 2 ? 1 : sg.n_tiles >= kQuarterTiles ? 2 : 3;
    const int rt = mode == 0 ? (w & 3) : mode == 1 ? (w & 1) : 0;
    const int ts = mode == 0 ? (w >> 2) : mode == 1 ? ((w >> 1) & 1) : mode == 2 ? (w & 3) : 0;
    const int sub0 = mode == 2 ? ts : 2 * ts;
    const bool act = 16 * rt < R;
    const bool last = c_t == sg.n_tiles - 1;
    unsigned char* stage = st_lds + (n & 1) * kStageBytes;
    if (c_t == 0) {
      m_run = -INFINITY;
      l_run = 0.f;
#pragma unroll
      for (int mt = 0; mt < 8; ++mt) o_acc[mt] = v4f{0.f, 0.f, 0.f, 0.f};
      if (act) {
        const unsigned char* qs = stage + 2 * kKvBytes + rt * 4096;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) qf[ks] = *reinterpret_cast<const v8s*>(qs + koff[ks]);
      }
    }
    if (act) {
      const int valid = min(kTok, sg.tok_count - c_t * kTok);
      const int vr = row_limit(valid, vis_lds[c_s], 16 * rt + lc, g, sg.tok_begin + c_t * kTok);
      const unsigned char* kt = stage + sub0 * 4096;
      const unsigned char* vt = stage + kKvBytes + sub0 * 4096;
      if (mode == 0)
        tile_compute<T, 2, 8>(kt, vt, qf, koff, voff8, sub0 * 16, vr, lg, scale, m_run, l_run, o_acc);
      else if (mode == 1)
        tile_compute<T, 2, 4>(kt, vt, qf, koff, voff4, sub0 * 16, vr, lg, scale, m_run, l_run, o_acc);
      else if (mode == 2)
        tile_compute<T, 1, 4>(kt, vt, qf, koff, voff4, sub0 * 16, vr, lg, scale, m_run, l_run, o_acc);
      else
        tile_compute<T, 4, 1>(kt, vt, qf, koff, voff1, 0, vr, lg, scale, m_run, l_run, o_acc);
    }

    if (last) {
      float l = l_run;
      l = rows4_sum(l);
      const int nmt = mode == 0 ? 8 : mode == 3 ? 1 : 4;
      const int mt0 = mode == 0 ? 0 : mode == 3 ? w : 4 * (w >> 2);
      // token-split waves hand their state to the ts == 0 wave of their (row
      // tile, head_dim part): o through this stage's K/V area (no loads target
      // it until the next iteration's barrier; at most 32 KB: 4 writers x 8 KB
      // in mode 0, writer w at 4 KB x w otherwise), m and l through ml_lds
      const int kslot = nmt * 1024;
      if (mode != 3) lds_sync();
      if (ts > 0 && act) {
        unsigned char* slot = stage + (mode == 0 ? w - 4 : w) * kslot;
#pragma unroll
        for (int mt = 0; mt < 8; ++mt)
          if (mt < nmt) *reinterpret_cast<v4f*>(slot + (mt * 64 + lane) * 16) = o_acc[mt];
        ml_lds[w * 128 + lane] = m_run;
        ml_lds[w * 128 + 64 + lane] = l;
      }
      if (mode != 3) lds_sync();
      if (ts == 0 && act) {
        const int np = mode == 2 ? 4 : mode == 3 ? 1 : 2;   // waves sharing the (row tile, head_dim part)
        for (int p = 1; p < np; ++p) {
          const int pw = mode == 0 ? w + 4 : mode == 1 ? w + 2 : w + p;   // partner wave
          const unsigned char* slot = stage + (mode == 0 ? pw - 4 : pw) * kslot;
          const float mb = ml_lds[pw * 128 + lane];
          const float lb = ml_lds[pw * 128 + 64 + lane];
          const float M = fmaxf(m_run, mb);
          const float ca = (M == -INFINITY) ? 0.f : exp2f(m_run - M);
          const float cb = (M == -INFINITY) ? 0.f : exp2f(mb - M);
          l = l * ca + lb * cb;
          m_run = M;
#pragma unroll
          for (int mt = 0; mt < 8; ++mt)
            if (mt < nmt)
              o_acc[mt] = o_acc[mt] * ca + *reinterpret_cast<const v4f*>(slot + (mt * 64 + lane) * 16) * cb;
        }
        // lane holds O^T[d = 16 (mt0 + mt) + 4 lg + i][row = 16 rt + lc]
        const int row = 16 * rt + lc;
        if (row < R) {
          const int j = row / g, hh = row - j * g, head = sg.head * g + hh;
          const int qi = sg.q_begin + j;
          const float inv = (l > 0.f) ? 1.f / l : 0.f;
          const float lse = (l > 0.f) ? (m_run + log2f(l)) * 0.69314718055994531f : -INFINITY;
          const int d0 = 16 * mt0 + 4 * lg;
          if (sg.out_slot < 0) {
            T* op = reinterpret_cast<T*>(a.out) + (int64_t)qi * a.o_sn + (int64_t)head * a.o_sh + d0;
#pragma unroll
            for (int mt = 0; mt < 8; ++mt)
              if (mt < nmt)
                __builtin_nontemporal_store(
                    pack4<T>(o_acc[mt][0] * inv, o_acc[mt][1] * inv, o_acc[mt][2] * inv, o_acc[mt][3] * inv),
                    reinterpret_cast<v4s*>(op + mt * 16));
            if (mt0 == 0 && lg == 0 && a.out_lse) __builtin_nontemporal_store(lse, a.out_lse + (int64_t)qi * a.hq + head);
          } else {
            const int64_t slot = (int64_t)(sg.out_slot + j) * g + hh;
            T* op = reinterpret_cast<T*>(a.part_o) + slot * kD + d0;
#pragma unroll
            for (int mt = 0; mt < 8; ++mt)
              if (mt < nmt)
                store_wt(reinterpret_cast<v4s*>(op + mt * 16),
                         pack4<T>(o_acc[mt][0] * inv, o_acc[mt][1] * inv, o_acc[mt][2] * inv, o_acc[mt][3] * inv));
            if (mt0 == 0 && lg == 0) store_wt(a.part_lse + slot, lse);
          }
        }
      }
    }
    }
    advance(c_s, c_t, c_sg);
    if (n + 1 < n_tiles) store(nx, (n + 1) & 1);
    load(nx, n + 3 < n_tiles, page);
    lds_sync();                                      // tile n + 1 stored; stage n & 1 free
  };
  // (both iterations of a trip unconditional: on every path from a set's loads
  // to its stores the other set's loads come in between)
  int n = 0;
  for (; n + 1 < n_tiles; n += 2) {
    iteration(n, rb);
    iteration(n + 1, ra);
  }
  if (n < n_tiles) iteration(n, rb);
}

// One tail item — tail chunks of one (query, KV head) — attended by one wave in
// its 8 KB LDS area; the normalised output and lse of the g heads go to the
// item's partial slot.
static_assert(kWaves * 2 * 4096 <= kLdsStages, "per-wave tail areas fit the stage buffers");

template <typename T>
__device__ __forceinline__ void tail_item(const StreamArgs& a, unsigned char* area, int idx) {
  const int lane = threadIdx.x & 63, lg = lane >> 4, lc = lane & 15;
  const int g = a.g;
  const int32_t* ip = a.titems + (int64_t)idx * kRecWords;
  const int qi = rfl(ip[0]), h = rfl(ip[1]), t0 = rfl(ip[2]), slot = rfl(ip[4]);
  const int nt = min(rfl(ip[3]), kTailChunks);
  const int2 ent = lane < nt ? a.tails[t0 + lane] : int2{0, 0};
  float m_run = -INFINITY, l_run = 0.f;
  v4f o_acc[8];
#pragma unroll
  for (int mt = 0; mt < 8; ++mt) o_acc[mt] = v4f{0.f, 0.f, 0.f, 0.f};
  tail_chunks<T>(a.q, a.q_sn, a.q_sh, a.kv, a.page_size, a.hkv, g, qi, h, ent, nt, 0, 1, area, a.scale_log2,
                 m_run, l_run, o_acc);
  float l = l_run;
  l = rows4_sum(l);
  // lane holds O^T[d = 16 mt + 4 lg + i][row lc]; items have chunks, so l > 0
  if (lc < g) {
    const float inv = 1.f / l;
    const int64_t sl = (int64_t)slot * g + lc;
    T* op = reinterpret_cast<T*>(a.part_o) + sl * kD + 4 * lg;
#pragma unroll
    for (int mt = 0; mt < 8; ++mt)
      store_wt(reinterpret_cast<v4s*>(op + 16 * mt),
               pack4<T>(o_acc[mt][0] * inv, o_acc[mt][1] * inv, o_acc[mt][2] * inv, o_acc[mt][3] * inv));
    if (lg == 0) store_wt(a.part_lse + sl, (m_run + log2f(l)) * 0.69314718055994531f);
  }
}

// A workgroup of the tail role: wave w attends tail items w, w + 8, ... of
// its range.
template <typename T>
__device__ __forceinline__ void tail_body(const StreamArgs& a, unsigned char* st_lds, int first, int count) {
  const int w = rfl(threadIdx.x >> 6);
  for (int it = w; it < count; it += kWaves) tail_item<T>(a, st_lds + w * 8192, first + it);
}

// REGS: the register-staged loop (the planner's choice for launches whose
// largest workgroup run has at least kRegsMinTiles tiles), else the
// direct-load loop.  One loop per kernel keeps each kernel's registers to
// what that loop needs.
template <typename T, bool REGS>
__global__ __launch_bounds__(kThreads) void attn_stream_kernel(StreamArgs a) {
  __shared__ __attribute__((aligned(16))) unsigned char st_lds[(REGS ? kRegStages : kDmaStages) * kStageBytes];
  __shared__ StreamSeg seg_lds[kMaxSegs];
  __shared__ int vis_lds[kMaxSegs];           // per segment: causal base, or kNoCausalS
  __shared__ float ml_lds[kWaves * 128];      // epilogue exchange of m and l

  const int tid = threadIdx.x;
  const int4 wi = a.wg[blockIdx.x];
  const int n_segs = rfl(wi.y), n_tiles = rfl(wi.z), cls = rfl(wi.w);
  if (cls == kTailRole) {
    tail_body<T>(a, st_lds, rfl(wi.x), n_segs);
  } else if (n_tiles > 0) {
    {
      const int* src = reinterpret_cast<const int*>(a.segs + wi.x);
      int* dst = reinterpret_cast<int*>(seg_lds);
      for (int i = tid; i < n_segs * 8; i += kThreads) dst[i] = src[i];
      for (int i = tid; i < n_segs; i += kThreads) vis_lds[i] = a.seg_causal ? a.seg_causal[wi.x + i] : kNoCausalS;
    }
    __syncthreads();
    if constexpr (REGS) {
      if (cls == 0) stream_body_regs<T, 0>(a, st_lds, seg_lds, vis_lds, ml_lds, n_segs, n_tiles);
      else if (cls == 2) stream_body_regs<T, 2>(a, st_lds, seg_lds, vis_lds, ml_lds, n_segs, n_tiles);
      else stream_body_regs<T, -1>(a, st_lds, seg_lds, vis_lds, ml_lds, n_segs, n_tiles);
    } else {
      if (cls == 0) stream_body_dma<T, 0>(a, st_lds, seg_lds, vis_lds, ml_lds, n_segs, n_tiles);
      else if (cls == 2) stream_body_dma<T, 2>(a, st_lds, seg_lds, vis_lds, ml_lds, n_segs, n_tiles);
      else if (cls == kClassWide) stream_body_dma<T, kClassWide>(a, st_lds, seg_lds, vis_lds, ml_lds, n_segs, n_tiles);
      else if (cls == kClassWide256)
        stream_body_regs<T, kClassWide256>(a, st_lds, seg_lds, vis_lds, ml_lds, n_segs, n_tiles);
      else if (cls == kClassWide256Dma)
        stream_body_dma<T, kClassWide256>(a, st_lds, seg_lds, vis_lds, ml_lds, n_segs, n_tiles);
      else stream_body_dma<T, -1>(a, st_lds, seg_lds, vis_lds, ml_lds, n_segs, n_tiles);
    }
  }
}

// WPR waves per record (query, KV head), 4 / WPR records per workgroup.  The
// tail pass first attends the record's tail chunks — 16 tokens of one page
// each, from the query's short groups — as one online softmax (a token in two
// groups counts twice, as two separately merged groups would count it): wave
// w of a record takes chunks w, w + WPR, ...; K and V rows go from global
// memory through the wave's LDS area into the streaming kernel's tile step
// (S^T = K Q^T on v_mfma_f32_16x16x32, P.V on 16x16x16, rows = the g query
// heads).  The record's waves' states and its partial slots are then combined
// by log-sum-exp with a running max, one (head, 4 columns) entry per thread.
// Each wave keeps the K/V rows of its next two chunks in flight.  A record
// with neither tail chunks nor slots writes o = 0 and lse = -inf.
constexpr int kTailDepth = 2;                  // tail chunks in flight per wave (3 measured slower)
template <typename T, int WPR>
__global__ __launch_bounds__(256, 2) void tail_merge_kernel(TailMergeArgs m) {
  constexpr int RPB = 4 / WPR;                 // records per workgroup
  constexpr int RT = 64 * WPR;                 // threads per record
  constexpr int C4 = kD / 4;
  __shared__ __attribute__((aligned(16))) unsigned char tl_lds[4][2 * 4096];   // per wave: K and V chunk
  __shared__ float st_m[4][16], st_l[4][16];
  const int tid = threadIdx.x, wv = rfl(tid >> 6);
  const int lane = tid & 63, lg = lane >> 4, lc = lane & 15;
  const int rb = wv / WPR, sw = wv - rb * WPR;  // record of the workgroup, wave within the record
  const int rtid = tid - rb * RT;
  const int e = blockIdx.x * RPB + rb;
  // the record and the live count (fixed layouts) load together: a record
  // within the launch's capacity is in bounds whether or not it is live
  int qi = 0, h = 0, s0 = 0, n = 0, t0 = 0, nt = 0;
  if (e < m.n_recs) {
    const int32_t* rp = m.recs + (int64_t)e * kRecWords;
    qi = rfl(rp[0]); h = rfl(rp[1]); s0 = rfl(rp[2]); n = rfl(rp[3]); t0 = rfl(rp[4]);
    nt = min(rfl(rp[5]), kTailChunks);
  }
  const int live = m.live ? *m.live : m.n_recs;
  if (WPR == 4 && e >= live) return;           // (one record per workgroup: uniform)
  const bool act = e < live;
  if (!act) n = nt = 0;
  const int g = m.g;
  const int32_t* slots = m.rec_slots + s0;
  // every wave holds all tail entries and the first 64 slot ids, lane k entry k
  const int2 ent = lane < nt ? m.tails[t0 + lane] : int2{0, 0};
  const int sid = lane < n ? slots[lane] : -1;

  // a batch of 8 slots of one (head, 4 columns) entry: o stays in its 16-bit
  // form until folded
  auto load_batch = [&](int hh, int d4, int k0, int (&sl)[8], float (&lv)[8], v4s (&ov)[8]) {
#pragma unroll
    for (int j = 0; j < 8; ++j)
      sl[j] = (k0 + j >= n) ? -1 : (k0 + j < 64) ? __builtin_amdgcn_readlane(sid, k0 + j) : slots[k0 + j];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (sl[j] >= 0) {
        const int64_t s = (int64_t)sl[j] * g + hh;
        lv[j] = m.part_lse[s];
        ov[j] = *reinterpret_cast<const v4s*>(reinterpret_cast<const T*>(m.part_o) + s * kD + 4 * d4);
      } else {
        lv[j] = -INFINITY;
        ov[j] = v4s{0, 0, 0, 0};
      }
    }
  };
  // this thread's first entry (its only one for g <= 4 with two or more waves
  // per record): its first slot batch loads now, beside the tail pass's K/V
  // loads, instead of after it
  const int ne = g * (kD / 4);
  const int ca = rtid;
  int sla[8];
  float lva[8];
  v4s ova[8];
  if (ca < ne) load_batch(ca / (kD / 4), ca % (kD / 4), 0, sla, lva, ova);

  float* part = reinterpret_cast<float*>(&tl_lds[0][0]);       // after the tail pass: [4][16][kD]
  float m_run = -INFINITY, l_run = 0.f;
  v4f o_acc[8];
#pragma unroll
  for (int mt = 0; mt < 8; ++mt) o_acc[mt] = v4f{0.f, 0.f, 0.f, 0.f};
  if (nt > 0) {
    tail_chunks<T, kTailDepth>(m.q, m.q_sn, m.q_sh, m.kv, m.page_size, m.hkv, g, qi, h, ent, nt, sw, WPR, tl_lds[wv],
                   m.scale_log2, m_run, l_run, o_acc);
    float l = l_run;
    l = rows4_sum(l);
    // lane holds O^T[d = 16 mt + 4 lg + i][row lc] (unnormalised, log2 domain); the
    // wave's state goes to its own K/V area
    if (lc < g) {
#pragma unroll
      for (int mt = 0; mt < 8; ++mt)
        *reinterpret_cast<v4f*>(part + (wv * 16 + lc) * kD + 16 * mt + 4 * lg) = o_acc[mt];
      if (lg == 0) {
        st_m[wv][lc] = m_run;
        st_l[wv][lc] = l;
      }
    }
  }
  // the record's other waves read the states: every wave of the workgroup
  // (including those of an inactive record) passes this barrier
  if (WPR > 1) __syncthreads();
  if (!act) return;

  T* out = reinterpret_cast<T*>(m.out) + (int64_t)qi * m.o_sn;
  // one (head, 4 columns) entry: the waves' tail states from LDS, then the
  // partial slots in batches of 8 (the first batch loaded by the caller), then
  // the normalised output and lse
  auto merge_entry = [&](int c, float (&lv0)[8], v4s (&ov0)[8]) {
    const int hh = c / C4, d4 = c - hh * C4;
    const int head = h * g + hh;
    float M = -INFINITY, z = 0.f;
    v4f acc = {0.f, 0.f, 0.f, 0.f};
    if (nt > 0) {
      float mw = -INFINITY;
#pragma unroll
      for (int w = 0; w < WPR; ++w) mw = fmaxf(mw, st_m[rb * WPR + w][hh]);
      float zt = 0.f;
      v4f at = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int w = 0; w < WPR; ++w) {
        const int ww = rb * WPR + w;
        const float mk = st_m[ww][hh];
        if (mk != -INFINITY) {
          const float sc = __builtin_amdgcn_exp2f(mk - mw);
          zt += st_l[ww][hh] * sc;
          at += *reinterpret_cast<const v4f*>(part + (ww * 16 + hh) * kD + 4 * d4) * sc;
        }
      }
      // the tail chunks hold a valid token, so zt > 0
      M = (mw + log2f(zt)) * 0.69314718055994531f;
      z = 1.f;
      acc = at * (1.f / zt);
    }
    auto fold = [&](const float (&lv)[8], const v4s (&ov)[8]) {
      float mx = M;
#pragma unroll
      for (int j = 0; j < 8; ++j) mx = fmaxf(mx, lv[j]);
      if (mx != -INFINITY) {
        const float sc = (M == -INFINITY) ? 0.f : expf(M - mx);
        z *= sc;
        acc *= sc;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float wgt = (lv[j] == -INFINITY) ? 0.f : expf(lv[j] - mx);
          z += wgt;
          acc += unpack4<T>(ov[j]) * wgt;
        }
        M = mx;
      }
    };
    fold(lv0, ov0);
    for (int k0 = 8; k0 < n; k0 += 8) {
      int sl[8];
      float lv[8];
      v4s ov[8];
      load_batch(hh, d4, k0, sl, lv, ov);
      fold(lv, ov);
    }
    const float inv = (z > 0.f) ? 1.f / z : 0.f;
    __builtin_nontemporal_store(pack4<T>(acc[0] * inv, acc[1] * inv, acc[2] * inv, acc[3] * inv),
                                reinterpret_cast<v4s*>(out + (int64_t)head * m.o_sh + 4 * d4));
    if (d4 == 0 && m.out_lse)
      __builtin_nontemporal_store((z > 0.f) ? M + logf(z) : -INFINITY, m.out_lse + (int64_t)qi * m.hq + head);
  };
  // the first entry from its prefetched batch, then the others two at a time:
  // both first slot batches are loaded before either is folded, so their
  // latencies overlap
  if (ca < ne) merge_entry(ca, lva, ova);
  for (int c = rtid + RT; c < ne; c += 2 * RT) {
    const int c1 = c + RT;
    int sl0[8], sl1[8];
    float lv0[8], lv1[8];
    v4s ov0[8], ov1[8];
    load_batch(c / C4, c % C4, 0, sl0, lv0, ov0);
    if (c1 < ne) load_batch(c1 / C4, c1 % C4, 0, sl1, lv1, ov1);
    merge_entry(c, lv0, ov0);
    if (c1 < ne) merge_entry(c1, lv1, ov1);
  }
}

}  // namespace stream

using namespace stream;

// ================================================================== host: plan
bool stream_eligible(int dtype, int head_dim, int group, int page_size, int flags) {
  return (dtype == BE_BF16 || dtype == BE_F16) && head_dim == kD && group <= kSegRows && page_size % 16 == 0 &&
         !(flags & (BE_PLAN_FORCE_VALU | BE_PLAN_FUSED_MERGE | BE_PLAN_TILE_KERNEL));
}

int stream_plan(const std::vector<Group>& groups, const be_level* levels, int num_levels, int64_t total_pages,
                int num_queries, int hq, int hkv, int d, int page_size, int num_pages, int dtype, int num_cus,
                int flags, const be_plan_caps* caps, int32_t* out, int64_t cap, be_attn_plan_info* info) {
  // causal groups (BE_PLAN_CAUSAL, last level, more than one query): query
  // q0 + i of n sees the group's first kv_len - n + i + 1 tokens; such a
  // group's tasks stop at their last query's last visible token and carry the
  // unclamped count of their first query for the kernel's per-row limit
  auto is_causal = [&](const Group& gr) {
    return (flags & BE_PLAN_CAUSAL) && gr.level == num_levels - 1 && gr.q1 - gr.q0 > 1;
  };
  (void)d;
  (void)num_pages;
  (void)dtype;
  const int g = hq / hkv;
  const int q_tile = std::max(1, kSegRows / g);
  const int W = std::max(1, num_cus);

  std::vector<int32_t> all_pages((size_t)total_pages);
  {
    int64_t p = 0;
    for (int lv = 0; lv < num_levels; ++lv) {
      const be_level& L = levels[lv];
      const int np = L.num_groups ? L.kv_indptr[L.num_groups] : 0;
      if (np) memcpy(all_pages.data() + p, L.kv_indices, np * sizeof(int32_t));
      p += np;
    }
  }

  // ---- tail chunks: groups of <= kTailTokens tokens and <= kTailQueries
  // queries are attended by the merge kernel, 16 tokens (one page) per chunk,
  // while each query holds at most kTailChunks of them
  // (per query as CSR: a first pass picks the groups and counts each query's
  // chunks, a second lays them out in group order)
  std::vector<int> tail_cnt((size_t)num_queries + 1, 0);
  std::vector<char> is_tail(groups.size(), 0);
  if (!(flags & BE_PLAN_NO_TAIL) && page_size % 16 == 0 && g <= 16) {
    for (size_t gi = 0; gi < groups.size(); ++gi) {
      const Group& gr = groups[gi];
      if (gr.kv_len <= 0 || gr.q1 <= gr.q0 || gr.kv_len > kTailTokens || gr.q1 - gr.q0 > kTailQueries ||
          is_causal(gr))
        continue;
      const int nch = (int)ceil_div(gr.kv_len, 16);
      bool fits = true;
      for (int qi = gr.q0; qi < gr.q1; ++qi) fits = fits && tail_cnt[qi] + nch <= kTailChunks;
      if (!fits) continue;
      is_tail[gi] = 1;
      for (int qi = gr.q0; qi < gr.q1; ++qi) tail_cnt[qi] += nch;
    }
  }
  std::vector<int> tail_beg((size_t)num_queries + 1, 0);
  for (int qi = 0; qi < num_queries; ++qi) tail_beg[qi + 1] = tail_beg[qi] + tail_cnt[qi];
  std::vector<int2> tails((size_t)tail_beg[num_queries]);
  {
    std::vector<int> fill(tail_beg.begin(), tail_beg.end() - 1);
    for (size_t gi = 0; gi < groups.size(); ++gi) {
      if (!is_tail[gi]) continue;
      const Group& gr = groups[gi];
      const int nch = (int)ceil_div(gr.kv_len, 16);
      for (int qi = gr.q0; qi < gr.q1; ++qi)
        for (int c = 0; c < nch; ++c) {
          const int tok0 = 16 * c;
          const int page = all_pages[(size_t)gr.page_base + tok0 / page_size];
          const int valid = std::min(16, gr.kv_len - tok0);
          tails[fill[qi]++] = int2{page, (tok0 % page_size) | (valid << 16)};
        }
    }
  }
  auto n_tails_of = [&](int qi) { return tail_beg[qi + 1] - tail_beg[qi]; };

  // ---- tasks: (query tile of a group, KV head), in group order.  A long group
  // of more than 64 rows takes query tiles of up to 128 rows (wide roles), so
  // its tiles are read once per 128 rows instead of once per 64; such a tile
  // costs kWideTileCost (twice the MFMA work of a 64-row tile for the same bytes).
  // (Only where every workgroup's run is long: a wide segment loads its Q rows
  // into registers, which drains the load pipeline once per segment, and the
  // direct-load loop it runs in fills and drains slower than the
  // register-staged one.)
  bool wide = !(flags & BE_PLAN_NO_WIDE) && !caps;
  if (wide) {
    int64_t tiles64 = 0;
    for (size_t gi = 0; gi < groups.size(); ++gi) {
      const Group& gr = groups[gi];
      if (gr.kv_len <= 0 || gr.q1 <= gr.q0 || is_tail[gi]) continue;
      tiles64 += ceil_div(gr.kv_len, kTok) * ceil_div(gr.q1 - gr.q0, q_tile) * hkv;
    }
    wide = tiles64 >= (int64_t)kWideMinRun * W;
  }
  auto wide_group = [&](size_t gi) {
    const Group& gr = groups[gi];
    return wide && !is_tail[gi] && gr.kv_len > 0 && gr.q1 > gr.q0 && !is_causal(gr) &&
           (gr.q1 - gr.q0) * g > kSegRows && ceil_div(gr.kv_len, kTok) >= kWideMinTiles;
  };
  // 256-row tasks when every group that takes the wide roles has at least 256
  // rows (no wave of a 256-row workgroup then idles on a short group's task)
  bool wide256 = wide && !(flags & BE_PLAN_NO_WIDE256);
  if (wide256) {
    bool any = false;
    for (size_t gi = 0; gi < groups.size() && wide256; ++gi)
      if (wide_group(gi)) {
        any = true;
        wide256 = (groups[gi].q1 - groups[gi].q0) * g >= kWide256Rows;
      }
    wide256 = wide256 && any;
  }
  const int q_tile_w = std::max(1, (wide256 ? kWide256Rows : kWideRows) / g);
  const int wide_cost = wide256 ? kWide256TileCost : kWideTileCost;
  struct Task { int q0, qn, page_base, kv_len, head, tiles, tc, vis0, grp; };
  std::vector<Task> tasks;
  int64_t total = 0;
  bool any_causal = false;
  for (size_t gi = 0; gi < groups.size(); ++gi) {
    const Group& gr = groups[gi];
    if (gr.kv_len <= 0 || gr.q1 <= gr.q0 || is_tail[gi]) continue;
    const bool cz = is_causal(gr);
    any_causal = any_causal || cz;
    const bool w128 = wide_group(gi);
    const int qt = w128 ? q_tile_w : q_tile;
    const int tc = w128 ? wide_cost : 4;
    for (int qa = gr.q0; qa < gr.q1; qa += qt) {
      const int qn = std::min(qt, gr.q1 - qa);
      const int vis0 = cz ? gr.kv_len - (gr.q1 - gr.q0) + (qa - gr.q0) + 1 : kNoCausalS;
      const int kv = cz ? std::max(0, std::min(gr.kv_len, vis0 + qn - 1)) : gr.kv_len;
      if (kv <= 0) continue;                        // the tile's queries see nothing: zero records
      const int tiles = (int)ceil_div(kv, kTok);
      for (int h = 0; h < hkv; ++h) {
        tasks.push_back(Task{qa, qn, gr.page_base, kv, h, tiles, tc, vis0, (int)gi});
        total += tc * (int64_t)tiles + kSegCost;
      }
    }
  }
  std::vector<int32_t> seg_vis;                     // per segment: its task's vis0

  // ---- roles: the tail chunks run either in tail-role workgroups of this
  // kernel (one wave per (query, KV head) item) while the other workgroups
  // stream -- the split following the planner costs (4 per tile, kSegCost per
  // segment start, kTailUnit per chunk of one KV head) -- and the merge
  // kernel then only merges, or in the merge kernel, fused with the merge.
  // The launch shares HBM either way; what decides is the merge kernel.  With
  // many chunks per query (long short-group suffixes) its tail pass streams
  // them at the streaming kernel's rate and the tail role's extra merge-only
  // pass costs more than the overlap saves (MI355X: north-star 48.4 vs 51.8
  // us per launch, config 2 21.9 vs 22.7, 8 chunks per query); with few it is
  // a latency-bound stub and the tail role wins (e2e step 24.95 vs 23.0, 1.5
  // per query; config 5 205.3 vs 202.1, 1.2; in a fixed layout the e2e step
  // 25.1 vs 23.3).  When the tail chunks are as much work as most of the
  // streamed tiles, running them beside the stream rather than after it wins
  // too (config 3: tail chunks 0.82 of the streamed tokens, 25.25 vs 26.0 us;
  // north-star and config 2, 0.5 of them: 52.1 vs 49.9 and 23.1 vs 22.2).  So
  // by default: the tail role when a plan with streamed groups has at most
  // kTailRoleChunks per query, or tail work of at least two thirds of its
  // streamed tiles' (in the planner's units: 1 per chunk and KV head, 4 per
  // 64-token tile).  BE_PLAN_TAIL_ROLE forces it, BE_PLAN_NO_TAIL_ROLE forbids it.
  int64_t tail_cost = 0, tail_chunks = 0, tile_cost = 0;
  for (int qi = 0; qi < num_queries; ++qi) tail_chunks += n_tails_of(qi);
  tail_cost = tail_chunks * hkv * kTailUnit;
  for (const Task& t : tasks) tile_cost += 4 * (int64_t)t.tiles;
  const bool auto_tail = !tasks.empty() && !(flags & BE_PLAN_NO_TAIL_ROLE) &&
                         (tail_chunks <= (int64_t)kTailRoleChunks * num_queries || 3 * tail_cost >= 2 * tile_cost);
  const bool tail_role = tail_cost > 0 && ((flags & BE_PLAN_TAIL_ROLE) || auto_tail) && (tasks.empty() || W >= 2);
  int W_t = 0;
  if (tail_role) {
    if (tasks.empty()) {
      W_t = W;
    } else {
      W_t = (int)((int64_t)W * tail_cost / (tail_cost + total));
      W_t = std::min(std::max(W_t, 1), W - 1);
    }
  }
  const int W_s = W - W_t;                              // streaming workgroups: [0, W_s)

  // ---- balanced contiguous runs.  A run's share is, when it opens, the
  // remaining cost (tiles, task starts, and one split per remaining run
  // boundary) over the remaining runs; a tile joins the run unless it would
  // overshoot that share by more than half its cost.  balance() walks the
  // tasks of `list` in order, each costing mult x (tc per tile + kSegCost per
  // segment start; seg for the sibling sets of 256-row tasks), over n_runs
  // runs, calling piece(run, list entry, first tile, tiles, new segment) for
  // every piece; segs_of(run) is the run's segment count so far (at most
  // kMaxSegs).
  std::vector<StreamSeg> segs;
  std::vector<int4> wg(W, int4{0, 0, 0, 0});
  auto balance = [&](const std::vector<int>& list, int n_runs, int mult, int seg, auto&& piece,
                     auto&& segs_of) -> bool {
    std::vector<int64_t> suffix(list.size() + 1, 0);
    for (size_t i = list.size(); i-- > 0;)
      suffix[i] = suffix[i + 1] + mult * (tasks[list[i]].tc * (int64_t)tasks[list[i]].tiles + seg);
    const int64_t sc = (int64_t)mult * seg;
    int b = 0;
    int64_t used = 0, share = 0;
    auto open_run = [&](size_t li, int tile) {
      const Task& t = tasks[list[li]];
      const int64_t rem = suffix[li + 1] + mult * (t.tc * (int64_t)(t.tiles - tile)) + sc + (int64_t)(n_runs - 1 - b) * sc;
      share = ceil_div(rem, n_runs - b);
      used = 0;
    };
    bool first = true;
    for (size_t li = 0; li < list.size(); ++li) {
      const Task& t = tasks[list[li]];
      const int64_t tc = (int64_t)mult * t.tc;
      bool open = false;                 // a segment of this task is open in run b
      for (int tile = 0; tile < t.tiles;) {
        if (first) {
          open_run(li, tile);
          first = false;
        }
        for (;;) {
          const int64_t c = tc + (open ? 0 : sc);
          const bool room = used + c / 2 <= share && (open || segs_of(b) < kMaxSegs);
          if (room || b == n_runs - 1) break;
          ++b;
          open = false;
          open_run(li, tile);
        }
        const bool fresh = !open;
        if (fresh) {
          if (segs_of(b) >= kMaxSegs) return false;
          used += sc;
          open = true;
        }
        // this tile joins, and with it every following tile of the task that
        // passes the same test (tile j more joins while used + (j - 1) tc +
        // tc / 2 <= share; the last run takes all)
        int take = t.tiles - tile;
        if (b != n_runs - 1) {
          const int64_t slack = share - (used + tc) - tc / 2;
          const int64_t more = slack < 0 ? 0 : slack / tc + 1;
          take = (int)std::min<int64_t>(take, 1 + more);
        }
        piece(b, (int)li, tile, take, fresh);
        used += (int64_t)take * tc;
        tile += take;
      }
    }
    return true;
  };
  // one piece of task ti in workgroup b (b's segments are appended together)
  auto put = [&](int b, int ti, int tile, int take, bool fresh) {
    const Task& t = tasks[ti];
    if (fresh) {
      if (wg[b].y == 0) wg[b].x = (int)segs.size();
      StreamSeg sgm;
      sgm.q_begin = t.q0;
      sgm.q_count = t.qn;
      sgm.page_begin = t.page_base;
      sgm.tok_begin = tile * kTok;
      sgm.tok_count = 0;
      sgm.head = t.head;
      sgm.out_slot = -1;
      sgm.n_tiles = 0;
      segs.push_back(sgm);
      seg_vis.push_back(t.vis0);
      wg[b].y += 1;
    }
    StreamSeg& cur = segs.back();
    cur.n_tiles += take;
    cur.tok_count = std::min(t.kv_len - cur.tok_begin, cur.n_tiles * kTok);
    wg[b].z += take;
  };

  // Sibling sets: the k query tiles of one group and KV head read the same
  // K/V tiles.  When every group split into several tiles has the same k, its
  // sets are balanced as units over virtual runs, and virtual run v puts
  // sibling s in workgroup (v / 8) 8 k + 8 s + v % 8: the k workgroups of a
  // piece share an XCD (workgroups are dispatched to the 8 XCDs round-robin)
  // and read each tile at about the same time, so one of them fetches it from
  // HBM and the others find it in that XCD's L2 (config 5 with 1-token
  // suffixes on MI355X: 181-187 us per launch with the siblings aligned, 197
  // with them on different XCDs).  The other tasks fill the other workgroups.
  // Runs that are not sibling sets take the workgroups XCD by XCD (0, 8, 16,
  // ..., then 1, 9, ...): consecutive runs, which hold the pieces of one split
  // task, then share an XCD, and the pieces after the first find the task's
  // query rows in that XCD's L2.
  std::vector<int> xcd_order;
  xcd_order.reserve(W_s);
  for (int x = 0; x < 8; ++x)
    for (int b = x; b < W_s; b += 8) xcd_order.push_back(b);
  std::vector<std::vector<int>> sets;               // task indices, sibling order
  std::vector<char> in_set(tasks.size(), 0);
  int k_sib = 0;
  {
    std::vector<std::vector<int>> all;
    std::vector<int> set_of(groups.size() * (size_t)hkv, -1);
    for (size_t ti = 0; ti < tasks.size(); ++ti) {
      const Task& t = tasks[ti];
      int& si = set_of[(size_t)t.grp * hkv + t.head];
      if (si < 0) {
        si = (int)all.size();
        all.emplace_back();
      }
      all[si].push_back((int)ti);
    }
    for (auto& st : all) {
      if (st.size() < 2) continue;
      // siblings of a causal group see different token counts: not paired
      bool same = true;
      for (int ti : st) same = same && tasks[ti].tiles == tasks[st[0]].tiles && tasks[ti].vis0 == kNoCausalS;
      if (!same) continue;
      if (k_sib == 0) k_sib = (int)st.size();
      if ((int)st.size() != k_sib) {
        k_sib = -1;
        break;
      }
      sets.push_back(st);
    }
    if (k_sib < 2) sets.clear();
    for (const auto& st : sets)
      for (int ti : st) in_set[ti] = 1;
  }
  const int v_max = k_sib >= 2 ? 8 * (W_s / (8 * k_sib)) : 0;
  if (v_max > 0) {
    std::vector<int> set_list, rest_list;
    for (const auto& st : sets) set_list.push_back(st[0]);
    int64_t set_sum = 0, rest_sum = 0;
    const int set_seg = wide256 && tasks[set_list[0]].tc == kWide256TileCost ? kWide256SegCost : kSegCost;
    for (size_t ti = 0; ti < tasks.size(); ++ti) {
      const int64_t c = tasks[ti].tc * (int64_t)tasks[ti].tiles + kSegCost;
      if (in_set[ti]) set_sum += c - kSegCost + set_seg;
      else {
        rest_sum += c;
        rest_list.push_back((int)ti);
      }
    }
    // virtual runs: the split that best evens the two sides' cost per workgroup
    int V = v_max;
    if (!rest_list.empty()) {
      V = 1;
      int64_t best = INT64_MAX;
      for (int v = 1; v <= v_max && W_s - v * k_sib >= 1; ++v) {
        const int64_t a = ceil_div(set_sum, (int64_t)v * k_sib), c = ceil_div(rest_sum, (int64_t)(W_s - v * k_sib));
        if (std::max(a, c) < best) {
          best = std::max(a, c);
          V = v;
        }
      }
    }
    auto slot = [&](int v, int sib) { return (v / 8) * 8 * k_sib + 8 * sib + (v % 8); };
    struct Piece { int set, tile, take; };
    std::vector<std::vector<Piece>> vpieces(V);
    const bool ok = balance(
        set_list, V, k_sib, set_seg,
        [&](int v, int li, int tile, int take, bool fresh) {
          if (fresh) vpieces[v].push_back(Piece{li, tile, 0});
          vpieces[v].back().take += take;
        },
        [&](int v) { return (int)vpieces[v].size(); });
    if (!ok) return BE_ERR_UNSUPPORTED;
    std::vector<char> taken(W_s, 0);
    for (int v = 0; v < V; ++v)
      for (int sib = 0; sib < k_sib; ++sib) {
        const int b = slot(v, sib);
        taken[b] = 1;
        for (const Piece& pc : vpieces[v]) put(b, sets[pc.set][sib], pc.tile, pc.take, true);
      }
    std::vector<int> free_wg;
    for (int b : xcd_order)
      if (!taken[b]) free_wg.push_back(b);
    if (!rest_list.empty()) {
      const bool ok2 = balance(
          rest_list, (int)free_wg.size(), 1, kSegCost,
          [&](int r, int li, int tile, int take, bool fresh) { put(free_wg[r], rest_list[li], tile, take, fresh); },
          [&](int r) { return wg[free_wg[r]].y; });
      if (!ok2) return BE_ERR_UNSUPPORTED;
    }
  } else {
    std::vector<int> all(tasks.size());
    for (size_t ti = 0; ti < tasks.size(); ++ti) all[ti] = (int)ti;
    const bool ok = balance(
        all, W_s, 1, kSegCost,
        [&](int r, int li, int tile, int take, bool fresh) { put(xcd_order[r], li, tile, take, fresh); },
        [&](int r) { return wg[xcd_order[r]].y; });
    if (!ok) return BE_ERR_UNSUPPORTED;
  }

  // ---- class per workgroup: the wave-role mode every segment of the
  // workgroup takes (0 or 2, which have specialised loops), else kClassGeneric;
  // a workgroup holding a segment of more than 64 rows runs all of its
  // segments with the wide roles (class 5: 32 rows per wave).
  bool any_wide = false;
  for (int b = 0; b < W_s; ++b) {
    int cls = -2;
    bool big = false;
    for (int i = wg[b].x; i < wg[b].x + wg[b].y; ++i) {
      const StreamSeg& sgm = segs[i];
      const int nt = (sgm.q_count * g + 15) / 16;
      big = big || sgm.q_count * g > kSegRows;
      const int md = nt >= 3 ? 0 : nt == 2 ? 1 : sgm.n_tiles >= kQuarterTiles ? 2 : 3;
      cls = cls == -2 ? md : cls == md ? cls : -1;
    }
    wg[b].w = big ? (wide256 ? ((flags & BE_PLAN_NO_REGS) ? kClassWide256Dma : kClassWide256) : kClassWide)
                  : (cls == 0 || cls == 2) ? cls : kClassGeneric;
    any_wide = any_wide || big;
  }

  // ---- partial slots and merge records per (query, KV head).  Per KV head
  // (head-major rows of num_queries + 1): cnt, the segments covering each
  // query, from a difference array over the segments' query ranges; a segment
  // is written directly when every query it covers has one segment and no tail
  // chunks (a prefix count of the queries that fail this)
  const size_t nq1 = (size_t)num_queries + 1;
  std::vector<int> cnt((size_t)hkv * nq1, 0);
  for (const StreamSeg& s : segs) {
    cnt[(size_t)s.head * nq1 + s.q_begin] += 1;
    cnt[(size_t)s.head * nq1 + s.q_begin + s.q_count] -= 1;
  }
  std::vector<int> undirect((size_t)hkv * nq1, 0);
  for (int h = 0; h < hkv; ++h) {
    int* c = cnt.data() + (size_t)h * nq1;
    int* u = undirect.data() + (size_t)h * nq1;
    int run = 0;
    for (int qi = 0; qi < num_queries; ++qi) {
      run += c[qi];
      c[qi] = run;
      u[qi + 1] = u[qi] + ((run != 1 || n_tails_of(qi) != 0) ? 1 : 0);
    }
  }
  auto cnt_of = [&](int qi, int h) { return cnt[(size_t)h * nq1 + qi]; };
  int n_slots = 0;
  for (StreamSeg& s : segs) {
    const int* u = undirect.data() + (size_t)s.head * nq1;
    if (u[s.q_begin + s.q_count] != u[s.q_begin]) {
      s.out_slot = n_slots;
      n_slots += s.q_count;
    }
  }
  // tail items (tail role): up to kItemChunks tail chunks of one (query, KV
  // head), each with a slot
  std::vector<int32_t> titems;
  if (tail_role) {
    int t0 = 0;
    for (int qi = 0; qi < num_queries; ++qi) {
      const int nt = n_tails_of(qi);
      for (int h = 0; h < hkv; ++h)
        for (int c = 0; c < nt; c += kItemChunks) {
          const int32_t it[kRecWords] = {qi, h, t0 + c, std::min(kItemChunks, nt - c), n_slots, 0, 0, 0};
          titems.insert(titems.end(), it, it + kRecWords);
          ++n_slots;
        }
      t0 += nt;
    }
  }
  // slot ids per (query, KV head) as CSR: count, prefix, fill in segment order
  const size_t nqh = (size_t)num_queries * hkv;
  std::vector<int> sbeg(nqh + 1, 0);
  {
    // slot-bearing segments per (query, KV head): a difference array per head
    std::fill(undirect.begin(), undirect.end(), 0);
    for (const StreamSeg& s : segs)
      if (s.out_slot >= 0) {
        undirect[(size_t)s.head * nq1 + s.q_begin] += 1;
        undirect[(size_t)s.head * nq1 + s.q_begin + s.q_count] -= 1;
      }
    for (int h = 0; h < hkv; ++h) {
      int run = 0;
      for (int qi = 0; qi < num_queries; ++qi) {
        run += undirect[(size_t)h * nq1 + qi];
        sbeg[(size_t)qi * hkv + h + 1] = run;
      }
    }
  }
  for (size_t i = 0; i < titems.size(); i += kRecWords) sbeg[(size_t)titems[i] * hkv + titems[i + 1] + 1] += 1;
  for (size_t k = 0; k < nqh; ++k) sbeg[k + 1] += sbeg[k];
  std::vector<int> slot_ids((size_t)sbeg[nqh]);
  {
    std::vector<int> fill(sbeg.begin(), sbeg.end() - 1);
    for (const StreamSeg& s : segs)
      if (s.out_slot >= 0)
        for (int j = 0; j < s.q_count; ++j) slot_ids[fill[(size_t)(s.q_begin + j) * hkv + s.head]++] = s.out_slot + j;
    for (size_t i = 0; i < titems.size(); i += kRecWords)
      slot_ids[fill[(size_t)titems[i] * hkv + titems[i + 1]]++] = titems[i + 4];
  }
  // records (query, KV head) in query order; a record's slots are its CSR
  // range of slot_ids, which is already in record order
  std::vector<int32_t> recs(nqh * kRecWords);
  int64_t n_recs = 0;
  for (int qi = 0; qi < num_queries; ++qi) {
    const int t0 = tail_beg[qi], nt_q = n_tails_of(qi);
    const int nt = tail_role ? 0 : nt_q;                 // tail role: the chunks arrive as slots
    for (int h = 0; h < hkv; ++h) {
      const size_t k = (size_t)qi * hkv + h;
      const int ns = sbeg[k + 1] - sbeg[k];
      if (cnt_of(qi, h) == 1 && nt_q == 0 && ns == 0) continue;   // written directly
      int32_t* r = recs.data() + n_recs * kRecWords;
      r[0] = qi;
      r[1] = h;
      r[2] = sbeg[k];
      r[3] = ns;
      r[4] = t0;
      r[5] = nt;
      r[6] = 0;
      r[7] = 0;
      ++n_recs;
    }
  }
  const std::vector<int>& rec_slots = slot_ids;
  const int64_t n_tails = (int64_t)tails.size();
  const int64_t n_items = (int64_t)titems.size() / kRecWords;
  if (tail_role) {
    // contiguous item ranges over the tail workgroups, balanced by chunks
    int64_t left = 0;
    for (int64_t i = 0; i < n_items; ++i) left += titems[i * kRecWords + 3];
    int64_t i = 0;
    for (int b = W_s; b < W; ++b) {
      const int64_t share = ceil_div(left, W - b);
      int64_t got = 0;
      wg[b] = int4{(int)i, 0, 0, kTailRole};
      while (i < n_items && (got == 0 || got + titems[i * kRecWords + 3] / 2 <= share || b == W - 1)) {
        got += titems[i * kRecWords + 3];
        ++i;
        wg[b].y += 1;
      }
      left -= got;
    }
  }

  // ---- serialise: header, workgroup table, segments, pages, records, record
  // slots, tail chunks
  const int64_t n_segs = (int64_t)segs.size();
  if (caps) {
    if (n_segs > caps->max_items || total_pages > caps->max_pages || n_recs > caps->max_merge ||
        n_slots > caps->max_merge_rows || n_tails > caps->max_tails || n_items > caps->max_tails)
      return fail(BE_ERR_CAPACITY,
                  "plan exceeds its fixed capacities: segments %lld/%d pages %lld/%d records %lld/%d slots %d/%d "
                  "tail chunks %lld/%d",
                  (long long)n_segs, caps->max_items, (long long)total_pages, caps->max_pages, (long long)n_recs,
                  caps->max_merge, n_slots, caps->max_merge_rows, (long long)n_tails, caps->max_tails);
  }
  const int64_t c_segs = caps ? caps->max_items : n_segs;
  const int64_t c_pages = caps ? caps->max_pages : total_pages;
  const int64_t c_recs = caps ? caps->max_merge : n_recs;
  const int64_t c_slots = caps ? caps->max_merge_rows : n_slots;
  const int64_t c_tails = caps ? caps->max_tails : n_tails;
  int64_t off = kPlanHeader;
  const int64_t off_wg = off;     off += 4 * (int64_t)W;
  const int64_t off_segs = off;   off += 8 * c_segs;
  const int64_t off_pages = off;  off += c_pages;
  const int64_t off_recs = off;   off += kRecWords * c_recs;
  const int64_t off_rslots = off; off += c_slots;
  off = ceil_div(off, 2) * 2;
  const int64_t off_tails = off;  off += 2 * c_tails;
  const int64_t c_items = caps ? (int64_t)caps->max_tails : n_items;   // an item holds >= 1 tail chunk
  const int64_t off_items = off;  off += kRecWords * c_items;
  const int64_t off_causal = off; off += any_causal ? c_segs : 0;
  off = ceil_div(off, 4) * 4;
  if (off > cap || off > INT32_MAX) {
    info->plan_ints = (int32_t)std::min<int64_t>(off, INT32_MAX);   // the words needed (0: a capacity of caps)
    return fail(BE_ERR_CAPACITY, "plan needs %lld int32 words, buffer holds %lld", (long long)off, (long long)cap);
  }
  if (any_causal && n_segs) memcpy(out + off_causal, seg_vis.data(), n_segs * sizeof(int32_t));
  for (int i = 0; i < kPlanHeader; ++i) out[i] = 0;
  out[kHdrItems] = (int32_t)n_segs;
  out[kHdrMerge] = (int32_t)n_recs;
  out[kHdrRows] = n_slots;
  out[kHdrTailItems] = (int32_t)n_items;
  memcpy(out + off_wg, wg.data(), wg.size() * sizeof(int4));
  if (n_segs) memcpy(out + off_segs, segs.data(), n_segs * sizeof(StreamSeg));
  if (total_pages) memcpy(out + off_pages, all_pages.data(), total_pages * sizeof(int32_t));
  if (n_recs) memcpy(out + off_recs, recs.data(), n_recs * kRecWords * sizeof(int32_t));
  if (!rec_slots.empty()) memcpy(out + off_rslots, rec_slots.data(), rec_slots.size() * sizeof(int32_t));
  if (n_tails) memcpy(out + off_tails, tails.data(), n_tails * sizeof(int2));
  if (n_items) memcpy(out + off_items, titems.data(), titems.size() * sizeof(int32_t));

  info->num_items = (int32_t)n_segs;
  info->num_part_rows = n_slots;
  info->num_merge = (int32_t)n_recs;
  info->num_queries = num_queries;
  info->kernel = 2;
  info->tile_rows = kSegRows;
  info->chunk_tokens = (int32_t)std::min<int64_t>(INT32_MAX, ceil_div(total, 4 * (int64_t)W) * kTok);
  info->plan_ints = (int32_t)off;
  info->off_items = (int32_t)off_segs;
  info->off_pages = (int32_t)off_pages;
  info->off_merge_q = (int32_t)off_recs;
  info->off_merge_rows = (int32_t)off_rslots;
  info->static_layout = caps ? 1 : 0;
  info->grid_items = W;
  info->grid_merge = (int32_t)c_recs;
  info->part_rows_cap = (int32_t)c_slots;
  info->counter_offset = ceil_div(c_slots * g * (kD * 2 + 4), 256) * 256;   // 16-bit o, fp32 lse
  info->counter_bytes = 0;
  info->partial_bytes = info->counter_offset;
  info->num_wg = W;
  info->off_wg = (int32_t)off_wg;
  info->off_seg_causal = any_causal ? (int32_t)off_causal : 0;
  info->off_records = (int32_t)off_recs;
  info->off_record_slots = (int32_t)off_rslots;
  info->num_tails = (int32_t)n_tails;
  info->off_tails = (int32_t)off_tails;
  info->num_tail_items = (int32_t)n_items;
  info->off_tail_items = (int32_t)off_items;
  // the loop: register-staged once the largest workgroup run is long enough
  // for its faster steady state to outweigh its slower fill and drain (fixed
  // layouts, whose runs change between plans of one layout, keep the
  // direct-load loop so that a captured launch stays valid)
  int max_tiles = 0;
  for (int b = 0; b < W; ++b) max_tiles = std::max(max_tiles, wg[b].w == kTailRole ? 0 : wg[b].z);
  // (wide roles run in the direct-load loop only)
  info->stream_loop = (!caps && !any_wide && !(flags & BE_PLAN_NO_REGS) && max_tiles >= kRegsMinTiles) ? 1 : 0;
  {
    // waves per record of the tail-and-merge kernel while all of them stay
    // resident at once (two waves per SIMD, 8 per CU): 4 where the records'
    // tails are long enough to share out, else 2 (a record's second wave
    // halves its merge of slots, whether or not it has tail chunks: 22.0 vs
    // 24.2 us at the e2e shape on MI355X), else 1.  A fixed layout keeps one
    // launch shape for every plan: 2.
    int64_t chunks = 0;
    for (int64_t r = 0; r < n_recs; ++r) chunks += recs[r * kRecWords + 5];
    const int64_t slots8 = 8 * (int64_t)W;
    info->tail_waves = caps ? 2
                       : (n_recs > 0 && 4 * n_recs <= slots8 && chunks >= 4 * n_recs) ? 4
                       : (n_recs > 0 && 2 * n_recs <= slots8)                          ? 2
                                                                                      : 1;
  }
  return BE_OK;
}

// ================================================================== host: run
int stream_run(const be_attn_plan_info* info, const int32_t* plan, void* partials, const void* q, int64_t q_sn,
               int64_t q_sh, const void* kv, void* out, int64_t o_sn, int64_t o_sh, float* lse, float sm_scale,
               int phases, hipStream_t st) {
  const int hq = info->num_qo_heads, hkv = info->num_kv_heads, g = hq / hkv;
  BE_REQUIRE(info->head_dim == kD, "corrupt plan info: streaming kernel with head_dim %d", info->head_dim);
  BE_REQUIRE((reinterpret_cast<uintptr_t>(q) & 15) == 0 && q_sn % 8 == 0 && q_sh % 8 == 0,
             "q must be 16-byte aligned with strides that are multiples of 8 elements");
  BE_REQUIRE((reinterpret_cast<uintptr_t>(out) & 7) == 0 && o_sn % 4 == 0 && o_sh % 4 == 0,
             "out must be 8-byte aligned with strides that are multiples of 4 elements");
  void* part_o = partials;
  float* part_lse = partials ? reinterpret_cast<float*>(static_cast<char*>(partials) +
                                                        (int64_t)info->part_rows_cap * g * kD * 2)
                             : nullptr;
  const int ps = info->page_size;
  if ((phases & BE_RUN_ATTENTION) && info->num_wg > 0 &&
      (info->static_layout || info->num_items > 0 || info->num_tail_items > 0)) {
    StreamArgs a;
    a.q = q; a.q_sn = q_sn; a.q_sh = q_sh;
    a.kv = kv;
    a.out = out; a.o_sn = o_sn; a.o_sh = o_sh; a.out_lse = lse;
    a.part_o = part_o; a.part_lse = part_lse;
    a.wg = reinterpret_cast<const int4*>(plan + info->off_wg);
    a.segs = reinterpret_cast<const StreamSeg*>(plan + info->off_items);
    a.seg_causal = info->off_seg_causal ? plan + info->off_seg_causal : nullptr;
    a.titems = plan + info->off_tail_items;
    a.tails = reinterpret_cast<const int2*>(plan + info->off_tails);
    a.pages = plan + info->off_pages;
    a.page_size = ps;
    a.page_shift = (ps & (ps - 1)) == 0 ? __builtin_ctz((unsigned)ps) : -1;
    a.hkv = hkv; a.hq = hq; a.g = g;
    a.scale_log2 = sm_scale * 1.4426950408889634f;
    const bool regs = info->stream_loop == 1;
    if (info->dtype == BE_BF16) {
      if (regs) attn_stream_kernel<bf16_t, true><<<info->num_wg, kThreads, 0, st>>>(a);
      else attn_stream_kernel<bf16_t, false><<<info->num_wg, kThreads, 0, st>>>(a);
    } else if (info->dtype == BE_F16) {
      if (regs) attn_stream_kernel<f16_t, true><<<info->num_wg, kThreads, 0, st>>>(a);
      else attn_stream_kernel<f16_t, false><<<info->num_wg, kThreads, 0, st>>>(a);
    }
    else return fail(BE_ERR_INVALID, "corrupt plan info: streaming kernel with dtype %d", info->dtype);
    BE_HIP_CHECK(hipGetLastError());
  }
  if ((phases & BE_RUN_MERGE) && info->grid_merge > 0) {
    TailMergeArgs m;
    m.part_o = part_o; m.part_lse = part_lse;
    m.recs = plan + info->off_records;
    m.rec_slots = plan + info->off_record_slots;
    m.tails = reinterpret_cast<const int2*>(plan + info->off_tails);
    m.live = info->static_layout ? plan + kHdrMerge : nullptr;
    m.q = q; m.q_sn = q_sn; m.q_sh = q_sh;
    m.kv = kv;
    m.out = out; m.o_sn = o_sn; m.o_sh = o_sh; m.out_lse = lse;
    m.n_recs = info->grid_merge; m.g = g; m.hq = hq; m.hkv = hkv; m.page_size = ps;
    m.scale_log2 = sm_scale * 1.4426950408889634f;
    // several waves per record where records are few and their tails long enough
    // to share out (tail_waves from the planner), four records per workgroup
    // with one wave each otherwise
    const int wpr = info->tail_waves;
    const int grid = (int)ceil_div(info->grid_merge, 4 / wpr);
    if (info->dtype == BE_BF16) {
      if (wpr == 4) tail_merge_kernel<bf16_t, 4><<<grid, 256, 0, st>>>(m);
      else if (wpr == 2) tail_merge_kernel<bf16_t, 2><<<grid, 256, 0, st>>>(m);
      else tail_merge_kernel<bf16_t, 1><<<grid, 256, 0, st>>>(m);
    } else {
      if (wpr == 4) tail_merge_kernel<f16_t, 4><<<grid, 256, 0, st>>>(m);
      else if (wpr == 2) tail_merge_kernel<f16_t, 2><<<grid, 256, 0, st>>>(m);
      else tail_merge_kernel<f16_t, 1><<<grid, 256, 0, st>>>(m);
    }
    BE_HIP_CHECK(hipGetLastError());
  }
  return BE_OK;
}

}  // namespace be

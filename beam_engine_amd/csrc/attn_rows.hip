// Merge-free decode attention over row blocks, gfx950 (bf16 / fp16 KV, head_dim 128).
//
// The same quantities as every other path of be_attn_run -- for each query,
// softmax(s q K^T) V over the union of its cascade groups, merged by
// log-sum-exp (FlashInfer's MultiLevelCascadeAttentionWrapper as the
// reference runs it, models/modeling_llama.py:321-367) -- computed without
// partial slots and without a second kernel:
//
//  * A task is one block of at most 16 rows (consecutive queries of one
//    level-0 group x the GQA heads of one KV head) and all of that block's
//    groups on every level, in level order ("passes").  One workgroup runs one
//    task and writes the block's final outputs, so no partial result leaves
//    the workgroup.
//  * A group shared by several blocks (a request's prefix, read by each of its
//    blocks) is read by each of them.  The planner orders the tasks so that
//    blocks sharing their level-0 group get workgroup ids equal modulo 8:
//    workgroups are dispatched round-robin over MI355X's 8 XCDs, so those
//    blocks run on one XCD and the repeated reads hit its L2 (measured: four
//    readers of one chunk per XCD take the time of one).
//  * Eight waves, each an independent stream of 16-token sub-tiles: wave w
//    takes sub-tiles w, w + 8, ... of the task's sub-tile sequence (each pass
//    cut into 16-token pieces; a piece lies in one page because the page
//    size is a multiple of 16).  A wave moves its own K and V rows global ->
//    LDS with direct loads into its own stages (kStages deep), waits for them
//    with explicit vmcnt counts and computes from them with no workgroup
//    barrier; rows of the block outside a pass's group are masked (score
//    -inf).  The waves' online-softmax states are combined through LDS at the
//    end.
//  * S^T = K Q^T with v_mfma_f32_16x16x32 (Q in registers as the B operand,
//    loaded straight from global memory), O^T += V^T P^T with
//    v_mfma_f32_16x16x16 (V^T read with ds_read_b64_tr_b16): the per-wave tile
//    step of the streaming kernel, on one 16-token sub-tile.

#include <math.h>

#include <algorithm>
#include <vector>

#include "attention.h"
#include "stream_device.h"

namespace be {
namespace rows {

using namespace be::stream;

constexpr int kWaves = 8;                        // 2 per SIMD: one wave's MFMA / softmax latency hides under the other's
constexpr int kThreads = 64 * kWaves;
constexpr int kStages = 2;                       // sub-tiles per wave in LDS (kStages - 1 loads in flight)
constexpr int kSubBytes = 16 * kD * 2;           // 16 K (or V) rows of 256 bytes
constexpr int kStageBytes = 2 * kSubBytes;       // K + V of one sub-tile
constexpr int kLds = kWaves * kStages * kStageBytes;
constexpr int kBlockRows = 16;
constexpr int kTilesPerWave = 8 / kWaves;         // head_dim tiles each wave finishes in the combine
static_assert(kWaves * kTilesPerWave == 8, "the waves share the 8 head_dim tiles");
constexpr int kTaskWords = 8;                    // q0, queries, first pass, passes, KV head, sub-tiles, pages, 0
constexpr int kPassWords = 4;                    // first page entry, tokens, row mask, sub-tiles
constexpr int kMaxPasses = 64;                   // passes of one task (LDS table)
constexpr int kMaxTaskPages = 2048;              // page ids of one task (LDS table)
constexpr int kTableBytes = kMaxPasses * 4 * 4 + kMaxPasses * 4 + kMaxTaskPages * 4;
static_assert(kLds + kTableBytes <= 160 * 1024, "stages and tables fit the LDS");
static_assert(kWaves * (kBlockRows * kD + 2 * kBlockRows) * 4 <= kLds, "the combine fits the stages");

struct RowsArgs {
  const void* q;
  int64_t q_sn, q_sh;
  const void* kv;
  void* out;
  int64_t o_sn, o_sh;
  float* out_lse;
  const int32_t* tasks;     // [n][8], in workgroup order
  const int32_t* passes;    // [n][4]
  const int32_t* pages;
  int n_tasks, page_size, hkv, hq, g;
  float scale_log2;
};

typedef const __attribute__((address_space(4))) int32_t* const_i32_t;   // scalar (constant) loads

__device__ __forceinline__ int sld(const int32_t* p, int i) { return ((const_i32_t)(uintptr_t)p)[rfl(i)]; }

template <typename T>
__global__ __launch_bounds__(kThreads) void attn_rows_kernel(RowsArgs a) {
  __shared__ __align__(16) unsigned char lds[kLds];
  __shared__ int pass_lds[kMaxPasses][4];          // first page (index into page_lds), tokens, mask, sub-tiles
  __shared__ int page_lds[kMaxTaskPages];
  const int task = blockIdx.x;
  if (task >= a.n_tasks) return;
  const int* tk = a.tasks + (int64_t)task * kTaskWords;
  const int q0 = sld(tk, 0), nq = sld(tk, 1), pass0 = sld(tk, 2), npass = sld(tk, 3), head = sld(tk, 4);
  const int nsub = sld(tk, 5);
  const int tid = threadIdx.x, w = rfl(tid >> 6), lane = tid & 63, lg = lane >> 4, lc = lane & 15;
  // the task's pass records and page ids into LDS (the planner keeps them within the tables)
  if (tid < 64) {
    int pb = 0, tok = 0, msk = 0, ns = 0, np = 0;
    if (tid < npass) {
      const int* pr = a.passes + (int64_t)(pass0 + tid) * kPassWords;
      pb = pr[0];
      tok = pr[1];
      msk = pr[2];
      ns = pr[3];
      np = (tok + a.page_size - 1) / a.page_size;
    }
    // exclusive scan of the page counts over the wave
    int incl = np;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int u = __shfl_up(incl, o, 64);
      if (tid >= o) incl += u;
    }
    if (tid < npass) {
      pass_lds[tid][0] = incl - np;
      pass_lds[tid][1] = tok;
      pass_lds[tid][2] = msk;
      pass_lds[tid][3] = ns;
    }
    // page ids of pass p at page_lds[first .. first + np)
    for (int p = 0; p < npass; ++p) {
      const int npp = __shfl(np, p, 64), first = __shfl(incl - np, p, 64), src = __shfl(pb, p, 64);
      for (int i = tid; i < npp; i += 64) page_lds[first + i] = a.pages[src + i];
    }
  }
  __syncthreads();
  const int g = a.g, ps = a.page_size, hkv = a.hkv;
  const int rows = nq * g;
  const float scale = a.scale_log2;

  // Q rows as the MFMA B operand: lane (lg, lc) holds Q[row lc][32 ks + 8 lg .. + 7]
  v8s qf[4];
  {
    const bool ok = lc < rows;
    const int qi = q0 + (ok ? lc / g : 0), qh = head * g + (ok ? lc % g : 0);
    const T* qp = reinterpret_cast<const T*>(a.q) + (int64_t)qi * a.q_sn + (int64_t)qh * a.q_sh + 8 * lg;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const v8s z = {0, 0, 0, 0, 0, 0, 0, 0};
      qf[ks] = ok ? *reinterpret_cast<const v8s*>(qp + 32 * ks) : z;
    }
    // retire the Q loads here, before the first direct load: the compiler's
    // wait insertion cannot count the direct loads and would otherwise keep a
    // full vmcnt(0) wait for Q inside the loop, draining the pipeline
    __builtin_amdgcn_s_waitcnt(BE_VMCNT(0));
  }
  // per-lane LDS offsets of the operand reads inside a 16-token sub-tile
  uint32_t koff[4], voff[8];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) koff[ks] = lc * 256 + ((((ks << 2) | lg) ^ lc) << 4);
  {
    const int tl = 4 * lg + (lc >> 2), b1 = (lc >> 1) & 1, b0 = lc & 1;
#pragma unroll
    for (int mt = 0; mt < 8; ++mt) voff[mt] = (uint32_t)(tl * 256 + ((((2 * mt) | b1) ^ tl) << 4) + (b0 << 3));
  }
  const uint32_t wave_lds = lds_addr(lds) + (uint32_t)(w * kStages * kStageBytes);
  const unsigned char* wave_ptr = lds + w * kStages * kStageBytes;
  const int64_t head_off = (int64_t)head * kD * 2;                 // bytes
  const int64_t row_bytes = (int64_t)hkv * kD * 2;                 // one token row of all KV heads
  const int64_t plane = (int64_t)ps * row_bytes;                   // K plane -> V plane of a page
  const uint64_t kvb = reinterpret_cast<uint64_t>(a.kv);

  // cursors over this wave's sub-tiles w, w + kWaves, ...: pass index and the
  // sub-tile's index inside the pass
  const int mine = nsub > w ? (nsub - w + kWaves - 1) / kWaves : 0;
  int lp = 0, li = w, cp = 0, ci = w;
  auto settle = [&](int& p, int& i) {
    while (p < npass) {
      const int n = rfl(pass_lds[p][3]);
      if (i < n) break;
      i -= n;
      ++p;
    }
  };
  settle(lp, li);
  settle(cp, ci);

  // issue the 8 direct loads (4 K, 4 V) of the load cursor's sub-tile into stage s
  auto issue = [&](int s) {
    const int tok0 = li * 16;
    const int valid = min(16, rfl(pass_lds[lp][1]) - tok0);
    const int pg = rfl(page_lds[rfl(pass_lds[lp][0]) + tok0 / ps]);
    const int slot0 = tok0 % ps;
    const uint64_t kbase = kvb + (uint64_t)(((int64_t)pg * 2 * ps + slot0) * row_bytes + head_off);
    const uint32_t lk = wave_lds + (uint32_t)(s * kStageBytes);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 4 * i + lg;
      const uint32_t off = (uint32_t)(min(r, valid - 1) * row_bytes + ((lc ^ r) << 4));
      dma16_sv(kbase, off, lk + i * 1024);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 4 * i + lg;
      const uint32_t off = (uint32_t)(min(r, valid - 1) * row_bytes + ((lc ^ r) << 4));
      dma16_sv(kbase + (uint64_t)plane, off, lk + kSubBytes + i * 1024);
    }
    li += kWaves;
    settle(lp, li);
  };

  float m_run = -INFINITY, l_run = 0.f;
  v4f o_acc[8];
#pragma unroll
  for (int mt = 0; mt < 8; ++mt) o_acc[mt] = (v4f){0.f, 0.f, 0.f, 0.f};

  int issued = 0;
  for (; issued < kStages - 1 && issued < mine; ++issued) issue(issued % kStages);
  for (int n = 0; n < mine; ++n) {
    if (issued < mine) {
      issue(issued % kStages);
      ++issued;
    }
    wait_vmcnt(8 * (issued - n - 1));
    const int valid = min(16, rfl(pass_lds[cp][1]) - ci * 16);
    const int mask = rfl(pass_lds[cp][2]);
    const int vrow = ((mask >> lc) & 1) ? valid : 0;
    const unsigned char* kt = wave_ptr + (n % kStages) * kStageBytes;
    tile_compute<T, 1, 8>(kt, kt + kSubBytes, qf, koff, voff, 0, vrow, lg, scale, m_run, l_run, o_acc);
    ci += kWaves;
    settle(cp, ci);
  }

  // ---- combine the waves' (m, l, o) through LDS; wave w finishes head_dim
  // tiles kTilesPerWave w .. + kTilesPerWave - 1 of every row
  l_run = rows4_sum(l_run);
  __syncthreads();                                   // every wave's stage reads are done
  float* o_lds = reinterpret_cast<float*>(lds);      // [wave][mt][lane][4]
  float* m_lds = o_lds + kWaves * kBlockRows * kD;   // [wave][16]
  float* l_lds = m_lds + kWaves * kBlockRows;
#pragma unroll
  for (int mt = 0; mt < 8; ++mt) *reinterpret_cast<v4f*>(o_lds + ((w * 8 + mt) * 64 + lane) * 4) = o_acc[mt];
  if (lg == 0) {
    m_lds[w * kBlockRows + lc] = m_run;
    l_lds[w * kBlockRows + lc] = l_run;
  }
  __syncthreads();
  float M = -INFINITY;
#pragma unroll
  for (int v = 0; v < kWaves; ++v) M = fmaxf(M, m_lds[v * kBlockRows + lc]);
  float c[kWaves];
  float L = 0.f;
#pragma unroll
  for (int v = 0; v < kWaves; ++v) {
    c[v] = (M == -INFINITY) ? 0.f : exp2f(m_lds[v * kBlockRows + lc] - M);
    L += l_lds[v * kBlockRows + lc] * c[v];
  }
  if (lc < rows) {
    const int qi = q0 + lc / g, qh = head * g + lc % g;
    const float inv = (L > 0.f) ? 1.f / L : 0.f;
    T* op = reinterpret_cast<T*>(a.out) + (int64_t)qi * a.o_sn + (int64_t)qh * a.o_sh + 4 * lg;
#pragma unroll
    for (int t = 0; t < kTilesPerWave; ++t) {
      const int mt = kTilesPerWave * w + t;
      v4f o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int v = 0; v < kWaves; ++v) o += *reinterpret_cast<const v4f*>(o_lds + ((v * 8 + mt) * 64 + lane) * 4) * c[v];
      __builtin_nontemporal_store(pack4<T>(o[0] * inv, o[1] * inv, o[2] * inv, o[3] * inv),
                                  reinterpret_cast<v4s*>(op + mt * 16));
    }
    if (w == 0 && lg == 0 && a.out_lse) {
      const float lse = (L > 0.f) ? (M + log2f(L)) * 0.69314718055994531f : -INFINITY;
      __builtin_nontemporal_store(lse, a.out_lse + (int64_t)qi * a.hq + qh);
    }
  }
}

}  // namespace rows

bool rows_preferred(const std::vector<Group>& groups, int num_queries, int g, int num_cus) {
  (void)groups;
  (void)num_queries;
  (void)g;
  (void)num_cus;
  return false;
}

// ---------------------------------------------------------------- planner
// Tasks: every level-0 group is cut into blocks of at most 16 / g queries (at
// least one); a block's passes are, level by level, the groups holding any of
// its queries (with the mask of the block's rows in each).  Queries outside
// every level-0 group form their own blocks.  Tasks are (block, KV head),
// ordered so that the blocks of one level-0 group and head share an XCD.
int rows_plan(const std::vector<Group>& groups, const be_level* levels, int num_levels, int64_t total_pages,
              int num_queries, int hq, int hkv, int page_size, int num_cus, int32_t* out, int64_t cap,
              be_attn_plan_info* info) {
  using namespace rows;
  const int g = hq / hkv;
  const int qb = std::max(1, kBlockRows / g);
  // groups per level, in query order (qo_indptr is monotone within a level)
  std::vector<std::vector<const Group*>> by_level(num_levels);
  for (const Group& gr : groups)
    if (gr.q1 > gr.q0 && gr.kv_len > 0) by_level[gr.level].push_back(&gr);
  // blocks: cut at level-0 group boundaries
  struct Block { int q0, q1, key; };
  std::vector<Block> blocks;
  {
    std::vector<int> start_key(num_queries + 1, -1);
    int key = 0;
    int q = 0;
    const auto& l0 = by_level.empty() ? std::vector<const Group*>() : by_level[0];
    size_t gi = 0;
    while (q < num_queries) {
      while (gi < l0.size() && l0[gi]->q1 <= q) ++gi;
      int end, k;
      if (gi < l0.size() && l0[gi]->q0 <= q) {
        end = l0[gi]->q1;
        k = (int)gi;
      } else {
        end = (gi < l0.size()) ? l0[gi]->q0 : num_queries;
        k = -1 - q;                                   // queries outside every level-0 group
      }
      for (int b = q; b < end; b += qb) blocks.push_back(Block{b, std::min(end, b + qb), k});
      (void)key;
      q = end;
    }
  }
  // passes of every block
  std::vector<int32_t> passes;        // [n][4]
  std::vector<int32_t> bp0, bpn, bsub;
  std::vector<size_t> cursor(num_levels, 0);
  for (const Block& b : blocks) {
    bp0.push_back((int32_t)(passes.size() / kPassWords));
    int np = 0, ns = 0;
    for (int lv = 0; lv < num_levels; ++lv) {
      const auto& gl = by_level[lv];
      size_t& c = cursor[lv];
      while (c < gl.size() && gl[c]->q1 <= b.q0) ++c;
      for (size_t j = c; j < gl.size() && gl[j]->q0 < b.q1; ++j) {
        const Group* gr = gl[j];
        const int lo = std::max(b.q0, gr->q0), hi = std::min(b.q1, gr->q1);
        if (lo >= hi) continue;
        uint32_t mask = 0;
        for (int qi = lo; qi < hi; ++qi)
          for (int h = 0; h < g; ++h) mask |= 1u << ((qi - b.q0) * g + h);
        const int sub = (gr->kv_len + 15) / 16;
        passes.insert(passes.end(), {gr->page_base, gr->kv_len, (int32_t)mask, sub});
        ++np;
        ns += sub;
      }
    }
    bpn.push_back(np);
    bsub.push_back(ns);
    int64_t task_pages = 0;
    for (int k = bp0.back(); k < bp0.back() + np; ++k) task_pages += ceil_div(passes[k * kPassWords + 1], page_size);
    if (np > kMaxPasses || task_pages > kMaxTaskPages) return BE_ERR_UNSUPPORTED;
  }
  const int nb = (int)blocks.size();
  const int64_t n_tasks = (int64_t)nb * hkv;
  // XCD-aware order: workgroup ids x, x + 8, x + 16, ... run on XCD x.  Keys
  // (level-0 group, head) go whole to the lane with the most room left; a key
  // larger than any lane's room is split.
  constexpr int kXcd = 8;
  std::vector<int64_t> room(kXcd);
  for (int x = 0; x < kXcd; ++x) room[x] = n_tasks > x ? (n_tasks - x + kXcd - 1) / kXcd : 0;
  std::vector<std::vector<int64_t>> lane_tasks(kXcd);
  {
    int64_t t = 0;
    for (int h = 0; h < hkv; ++h) {
      int bi = 0;
      while (bi < nb) {
        int bj = bi;
        while (bj < nb && blocks[bj].key == blocks[bi].key) ++bj;
        int remaining = bj - bi;
        int at = bi;
        while (remaining > 0) {
          int best = 0;
          for (int x = 1; x < kXcd; ++x)
            if (room[x] > room[best]) best = x;
          const int take = (int)std::min<int64_t>(remaining, room[best]);
          for (int k = 0; k < take; ++k) lane_tasks[best].push_back((int64_t)(at + k) * hkv + h);
          room[best] -= take;
          at += take;
          remaining -= take;
          t += take;
        }
        bi = bj;
      }
    }
    (void)t;
  }
  // plan layout
  int64_t off = kPlanHeader;
  const int64_t off_tasks = off;  off += n_tasks * kTaskWords;
  const int64_t off_passes = off; off += (int64_t)passes.size();
  const int64_t off_pages = off;  off += total_pages;
  if (off > cap) {
    info->plan_ints = (int32_t)std::min<int64_t>(off, INT32_MAX);   // the words needed
    return fail(BE_ERR_CAPACITY, "rows plan needs %lld int32 words, buffer holds %lld", (long long)off,
                (long long)cap);
  }
  memset(out, 0, kPlanHeader * sizeof(int32_t));
  out[kHdrItems] = (int32_t)n_tasks;
  for (int x = 0; x < kXcd; ++x)
    for (size_t k = 0; k < lane_tasks[x].size(); ++k) {
      const int64_t wg = x + (int64_t)kXcd * (int64_t)k;
      const int64_t t = lane_tasks[x][k];
      const int bi = (int)(t / hkv), h = (int)(t % hkv);
      int32_t* rec = out + off_tasks + wg * kTaskWords;
      rec[0] = blocks[bi].q0;
      rec[1] = blocks[bi].q1 - blocks[bi].q0;
      rec[2] = bp0[bi];
      rec[3] = bpn[bi];
      rec[4] = h;
      rec[5] = bsub[bi];
      rec[6] = 0;
      rec[7] = 0;
    }
  if (!passes.empty()) memcpy(out + off_passes, passes.data(), passes.size() * sizeof(int32_t));
  {
    int64_t p = 0;
    for (int lv = 0; lv < num_levels; ++lv) {
      const be_level& L = levels[lv];
      const int np = L.num_groups ? L.kv_indptr[L.num_groups] : 0;
      if (np) memcpy(out + off_pages + p, L.kv_indices, np * sizeof(int32_t));
      p += np;
    }
  }
  info->kernel = 3;
  info->num_items = (int32_t)n_tasks;
  info->grid_items = (int32_t)n_tasks;
  info->num_queries = num_queries;
  info->plan_ints = (int32_t)off;
  info->off_items = (int32_t)off_tasks;
  info->off_merge_rows = (int32_t)off_passes;      // the pass records
  info->off_pages = (int32_t)off_pages;
  info->tile_rows = kBlockRows;
  info->num_wg = (int32_t)n_tasks;
  (void)num_cus;
  (void)page_size;
  return BE_OK;
}

int rows_run(const be_attn_plan_info* info, const int32_t* plan, const void* q, int64_t q_sn, int64_t q_sh,
             const void* kv, void* out, int64_t o_sn, int64_t o_sh, float* lse, float sm_scale, int phases,
             hipStream_t st) {
  using namespace rows;
  if (!(phases & BE_RUN_ATTENTION) || info->num_items == 0) return BE_OK;
  RowsArgs a;
  a.q = q; a.q_sn = q_sn; a.q_sh = q_sh;
  a.kv = kv; a.out = out; a.o_sn = o_sn; a.o_sh = o_sh; a.out_lse = lse;
  a.tasks = plan + info->off_items;
  a.passes = plan + info->off_merge_rows;
  a.pages = plan + info->off_pages;
  a.n_tasks = info->num_items;
  a.page_size = info->page_size;
  a.hkv = info->num_kv_heads;
  a.hq = info->num_qo_heads;
  a.g = info->num_qo_heads / info->num_kv_heads;
  a.scale_log2 = sm_scale * 1.4426950408889634f;
  switch (info->dtype) {
    case BE_BF16: attn_rows_kernel<bf16_t><<<info->num_items, kThreads, 0, st>>>(a); break;
    case BE_F16: attn_rows_kernel<f16_t><<<info->num_items, kThreads, 0, st>>>(a); break;
    default: return fail(BE_ERR_INVALID, "rows kernel needs 16-bit storage");
  }
  BE_HIP_CHECK(hipGetLastError());
  return BE_OK;
}

}  // namespace be

// Per-step attention metadata of a live beam trie, on the host (no device code).
//
// The reference builds its FlashInfer cascade index arrays by walking every
// candidate's root-to-leaf path in Python each decode step
// (src/beam_engine/beam_state.py:211-412, get_cascade_input).  The engine here
// keeps a flat node table of the trie (parent, page, token count, last token,
// alive), updated as the trie changes, and rebuilds the arrays from it in one
// pass over the nodes plus O(levels) per candidate:
//
//  * node ids follow creation order, so a parent's id is below its
//    children's and increasing id is a top-down order;
//  * a node's level is its parent's, plus one when the parent has more than
//    one live child (beam_state.py:236-256); a level segment is the chain of
//    only-children from the node that opened it;
//  * each candidate appears at every level 0..max: below its own level its
//    group is keyed by the branch point that closes that level, at and above
//    it by its leaf (beam_state.py:290-306); groups are ordered by their first
//    candidate (beam_state.py:323);
//  * a group's pages are its key node's segment in path order (repeated page
//    ids kept once), its last page length the key node's token count, minus
//    one when the key is the candidate's own leaf (beam_state.py:343-356).
//
// The same pass gives each candidate's query token, write location and
// position (beam.py:180-221).
//
// be_trie_levels builds the other strategies' levels from the same walk.
// Each attends every candidate to the tokens of its root-to-leaf path
// exactly once (the flat strategy's result; FastTree's intent,
// attention/fasttree/preparation.py:60-105), decomposed into shared passes
// over the segments above:
//
//  * segments are numbered as the candidates' paths first reach them
//    (candidates in order, each path top down), so a parent's number is below
//    its children's; a segment's children are listed in that order;
//  * an edge is "absorbed" when the child's pass also reads its parent's
//    (effective) tokens and the parent's pass stops serving the child's
//    candidates.  Flat absorbs every edge (one pass per candidate over its
//    path), split none (one pass per segment, merged); tree decides each edge
//    top down, parents first, children in order, by a cost model: this
//    build's fitted kernel costs, or FastTree's padded-tile model
//    (preparation.py:34-57 with the constants of metadata.py:12-38);
//  * a candidate's passes along its path are its levels 0, 1, ...; at each
//    level the candidates served by one segment form one group per run of
//    consecutive candidates, runs in candidate order, with empty groups for
//    candidates that have no pass at that level;
//  * auto prices flat, split and tree with the fitted costs and builds the
//    cheapest (the first of them on a tie).
// These rules, and the float arithmetic of the costs, follow the Python
// restatement in beam_engine_amd/beam_state.py (segment_tree, absorb_edges,
// tree_levels) and beam_engine_amd/picker.py operation for operation, so the
// two produce identical levels and choices.

#include <algorithm>
#include <vector>

#include "common.h"

namespace {

// The top-down walk of the node table that every strategy starts from.
struct TrieWalk {
  std::vector<int32_t> nchild, lvl, head, bp;
  std::vector<int64_t> pre;
  int max_page = -1;

  int run(const int32_t* parent, const int32_t* page, const int32_t* ntok, const uint8_t* alive, int num_nodes) {
    using be::fail;
    nchild.assign((size_t)num_nodes, 0);
    for (int n = 0; n < num_nodes; ++n) {
      if (!alive[n]) continue;
      const int p = parent[n];
      if (p >= 0) {
        if (p >= n) return fail(BE_ERR_INVALID, "node %d: parent %d is not older than the node", n, p);
        if (!alive[p]) return fail(BE_ERR_INVALID, "node %d: parent %d is not live", n, p);
        nchild[p] += 1;
      }
    }
    // level, segment head, branch point closing the previous level (the
    // chain of these gives the lower levels' keys), tokens above
    lvl.assign((size_t)num_nodes, 0);
    head.assign((size_t)num_nodes, 0);
    bp.assign((size_t)num_nodes, -1);
    pre.assign((size_t)num_nodes, 0);
    for (int n = 0; n < num_nodes; ++n) {
      if (!alive[n]) continue;
      if (page[n] < 0) return fail(BE_ERR_INVALID, "node %d: negative page id", n);
      max_page = std::max(max_page, page[n]);
      if (ntok[n] < 0) return fail(BE_ERR_INVALID, "node %d: negative token count", n);
      const int p = parent[n];
      if (p < 0) {
        lvl[n] = 0, head[n] = n, bp[n] = -1, pre[n] = 0;
      } else if (nchild[p] > 1) {
        lvl[n] = lvl[p] + 1, head[n] = n, bp[n] = p, pre[n] = pre[p] + ntok[p];
      } else {
        lvl[n] = lvl[p], head[n] = head[p], bp[n] = bp[p], pre[n] = pre[p] + ntok[p];
      }
    }
    return BE_OK;
  }
};

int check_inputs(const int32_t* parent, const int32_t* page, const int32_t* ntok, const int32_t* last_tok,
                 const uint8_t* alive, int num_nodes, const int32_t* leaves, int num_cands, const int32_t* out,
                 int64_t out_capacity) {
  using be::fail;
  if (num_nodes < 0 || num_cands < 0) return fail(BE_ERR_INVALID, "negative node or candidate count");
  if (num_cands > 0 && (!parent || !page || !ntok || !last_tok || !alive || !leaves))
    return fail(BE_ERR_INVALID, "null node table or leaf list");
  if (!out && out_capacity > 0) return fail(BE_ERR_INVALID, "null output buffer");
  for (int c = 0; c < num_cands; ++c) {
    const int f = leaves[c];
    if (f < 0 || f >= num_nodes || !alive[f]) return fail(BE_ERR_INVALID, "candidate %d: leaf %d is not live", c, f);
  }
  return BE_OK;
}

// The candidate block (query token, write page, write slot, position) and
// the copy into the caller's buffer.
int finish(std::vector<int32_t>& buf, const TrieWalk& w, const int32_t* page, const int32_t* ntok,
           const int32_t* last_tok, const int32_t* leaves, int num_cands, int32_t* out, int64_t out_capacity,
           int64_t* out_used) {
  using be::fail;
  buf[1] = (int32_t)buf.size();
  for (int c = 0; c < num_cands; ++c) buf.push_back(ntok[leaves[c]] > 0 ? last_tok[leaves[c]] : 0);
  for (int c = 0; c < num_cands; ++c) buf.push_back(page[leaves[c]]);
  for (int c = 0; c < num_cands; ++c) buf.push_back(ntok[leaves[c]] - 1);
  for (int c = 0; c < num_cands; ++c) {
    const int64_t pos = w.pre[leaves[c]] + ntok[leaves[c]] - 1;
    if (pos > INT32_MAX) return fail(BE_ERR_INVALID, "candidate %d: position %lld overflows int32", c, (long long)pos);
    buf.push_back((int32_t)pos);
  }
  if (out_used) *out_used = (int64_t)buf.size();
  if ((int64_t)buf.size() > out_capacity)
    return fail(BE_ERR_CAPACITY, "trie metadata needs %lld int32 words, buffer holds %lld", (long long)buf.size(),
                (long long)out_capacity);
  memcpy(out, buf.data(), buf.size() * sizeof(int32_t));
  return BE_OK;
}

// The pages of the segment that ends at node key, in path order, a page id
// repeated along the chain kept once (its first occurrence).
void chain_pages(const TrieWalk& w, const int32_t* parent, const int32_t* page, int key, std::vector<int32_t>& chain,
                 std::vector<int32_t>& seen, int& stamp, std::vector<int32_t>& out) {
  chain.clear();
  for (int x = key;; x = parent[x]) {
    chain.push_back(page[x]);
    if (x == w.head[key]) break;
  }
  ++stamp;
  for (size_t a = chain.size(); a-- > 0;) {
    if (seen[chain[a]] == stamp) continue;
    seen[chain[a]] = stamp;
    out.push_back(chain[a]);
  }
}

// ---------------------------------------------------------------- costs
constexpr int kTileTokens = 64, kSegRows = 64, kTailTokens = 128, kTailQueries = 4, kTailChunk = 16;
constexpr int64_t kWideMinTiles = 8, kWideMinTiles64 = 64 * 256;

struct Costs {
  const be_tree_model* m;
  int g, hkv;
  bool tail_ok;

  // one group of nq queries over `tokens` tokens, all KV heads
  double group(int64_t nq, int64_t tokens) const {
    if (nq <= 0 || tokens <= 0) return 0.0;
    if (tail_ok && tokens <= kTailTokens && nq <= kTailQueries)
      return (double)(nq * hkv * ((tokens + kTailChunk - 1) / kTailChunk)) * m->tail;
    const int64_t tiles = (tokens + kTileTokens - 1) / kTileTokens;
    int64_t rows = nq * g;
    double cost = 0.0;
    if (rows > kSegRows && tiles >= kWideMinTiles && (rows + kSegRows - 1) / kSegRows * tiles * hkv >= kWideMinTiles64) {
      // the planner's wide segments: 256 rows when the group has that many, else 128
      const int64_t wr = rows >= 256 ? 256 : 128;
      const double coef = rows >= 256 ? m->tile_w256 : m->tile_w128;
      while (rows > 0) {
        rows -= std::min<int64_t>(rows, wr);
        cost += (double)tiles * coef + m->seg;
      }
      return cost * hkv;
    }
    // a group's second and later 64-row query tiles read their K/V from the
    // L2 the first one filled (the planner places them on one XCD)
    bool first = true;
    while (rows > 0) {
      const int64_t r = std::min<int64_t>(rows, kSegRows);
      cost += (double)tiles * (first ? m->tile_nt[std::min<int64_t>(4, (r + 15) / 16) - 1] : m->tile_sib) + m->seg;
      rows -= r;
      first = false;
    }
    return cost * hkv;
  }
  double slots(int64_t nq) const { return (double)(nq * hkv) * m->slot; }

  // FastTree's padded-tile work: query tiles (64 / g, 16 / g), KV tiles 32
  double cmm(int64_t nq, int64_t nk) const {
    const int64_t qt1 = 16 / g;
    const int64_t tq = nq > qt1 ? 64 / g : qt1;
    const int64_t tk = 32;
    int64_t r = (nq - 1) % tq;
    if (r < 0) r += tq;                       // floor modulo
    const int64_t pad_q = tq - (r + 1);
    const int64_t pad_k = std::max<int64_t>(0, tk - nk);
    return m->alpha * (double)pad_q * (double)g * (double)nk + m->beta * (double)pad_k * (double)nq * (double)g;
  }

  bool absorb(int64_t nq_cur, int64_t nq_child, int64_t len_parent, int64_t len_child) const {
    if (m->edge_model == BE_EDGES_FASTTREE) {
      const double split_k = cmm(nq_cur, len_parent) + cmm(nq_child, len_child) + m->gamma * (double)nq_child;
      const double split_q = cmm(nq_cur - nq_child, len_parent) + cmm(nq_child, len_child + len_parent);
      return split_k > split_q;
    }
    const double split = group(nq_cur, len_parent) + group(nq_child, len_child) + slots(nq_child);
    const double absorb = group(nq_cur - nq_child, len_parent) + group(nq_child, len_child + len_parent);
    return absorb < split;
  }
};

// The segment tree of the live trie.
struct SegTree {
  std::vector<int32_t> key, par, tokens, npages, pg_off, nq;
  std::vector<int32_t> pages;                         // own pages, concatenated
  std::vector<int32_t> kid_off, kids;                 // children in numbering order (CSR)
  std::vector<int32_t> path_off, path;                // each candidate's segments, top down

  int size() const { return (int)key.size(); }
};

void build_segments(const TrieWalk& w, const int32_t* parent, const int32_t* page, const int32_t* ntok,
                    const int32_t* leaves, int num_cands, int num_nodes, int page_size, bool include_self,
                    SegTree& s) {
  std::vector<int32_t> seg_of((size_t)num_nodes, -1);
  std::vector<int32_t> seen((size_t)w.max_page + 1, -1), chain, keys;
  int stamp = 0;
  std::vector<std::vector<int32_t>> kids;
  s.path_off.assign(1, 0);
  for (int c = 0; c < num_cands; ++c) {
    const int f = leaves[c];
    keys.clear();
    for (int x = f; x >= 0; x = w.bp[x]) keys.push_back(x);
    int prev = -1;
    for (size_t a = keys.size(); a-- > 0;) {
      const int k = keys[a];
      int i = seg_of[k];
      if (i < 0) {
        i = seg_of[k] = s.size();
        s.key.push_back(k);
        s.par.push_back(prev);
        s.pg_off.push_back((int32_t)s.pages.size());
        chain_pages(w, parent, page, k, chain, seen, stamp, s.pages);
        const int np = (int)s.pages.size() - s.pg_off.back();
        const int last = (k == f && !include_self) ? std::max(0, ntok[k] - 1) : ntok[k];
        s.npages.push_back(np);
        s.tokens.push_back((np - 1) * page_size + last);
        s.nq.push_back(0);
        kids.emplace_back();
        if (prev >= 0) kids[prev].push_back(i);
      }
      s.nq[i] += 1;
      s.path.push_back(i);
      prev = i;
    }
    s.path_off.push_back((int32_t)s.path.size());
  }
  s.kid_off.assign(1, 0);
  for (auto& v : kids) {
    s.kids.insert(s.kids.end(), v.begin(), v.end());
    s.kid_off.push_back((int32_t)s.kids.size());
  }
}

// Edge decisions top down (parents first, children in order); teff: each
// segment's effective token count.
void absorb_edges(const SegTree& s, const Costs& cm, std::vector<uint8_t>& absorbed, std::vector<int64_t>& teff) {
  const int n = s.size();
  std::vector<int64_t> nq(s.nq.begin(), s.nq.end());
  teff.assign(s.tokens.begin(), s.tokens.end());
  absorbed.assign((size_t)n, 0);
  for (int k = 0; k < n; ++k)
    for (int j = s.kid_off[k]; j < s.kid_off[k + 1]; ++j) {
      const int ch = s.kids[j];
      const int64_t nch = s.nq[ch];
      if (cm.absorb(nq[k], nch, teff[k], s.tokens[ch])) {
        absorbed[ch] = 1;
        nq[k] -= nch;
        teff[ch] = s.tokens[ch] + teff[k];
      }
    }
}

// Modelled cost of one decomposition: each segment's pass over its effective
// tokens for the candidates it serves, plus a slot for every pass of a
// candidate beyond its first.
double decomposition_cost(const SegTree& s, const Costs& cm, const std::vector<uint8_t>& absorbed,
                          const std::vector<int64_t>& teff, int num_cands) {
  const int n = s.size();
  double total = cm.m->fixed;
  std::vector<int64_t> served(s.nq.begin(), s.nq.end());
  for (int k = 0; k < n; ++k)
    if (absorbed[k]) served[s.par[k]] -= s.nq[k];
  for (int k = 0; k < n; ++k) total += cm.group(served[k], teff[k]);
  int64_t extra = 0;
  for (int c = 0; c < num_cands; ++c) {
    int64_t passes = 0;
    for (int j = s.path_off[c]; j < s.path_off[c + 1]; ++j) {
      const int k = s.path[j];
      const bool skip = j + 1 < s.path_off[c + 1] && absorbed[s.path[j + 1]];
      if (teff[k] > 0 && !skip) ++passes;
    }
    extra += std::max<int64_t>(0, passes - 1);
  }
  return total + cm.slots(extra);
}

double flat_cost(const SegTree& s, const Costs& cm, int num_cands) {
  const int n = s.size();
  std::vector<int64_t> cum((size_t)n, 0);
  for (int k = 0; k < n; ++k) cum[k] = s.tokens[k] + (s.par[k] >= 0 ? cum[s.par[k]] : 0);
  double sum = 0.0;
  for (int c = 0; c < num_cands; ++c) sum += cm.group(1, cum[s.path[s.path_off[c + 1] - 1]]);
  return cm.m->fixed + sum;
}

// The level arrays of a decomposition, appended to buf with their records.
int emit_levels(const SegTree& s, const std::vector<uint8_t>& absorbed, int num_cands, int page_size,
                std::vector<int32_t>& buf) {
  const int n = s.size();
  // effective pages: the absorbed ancestors' pages, then the segment's own
  std::vector<int32_t> eff_off((size_t)n + 1, 0), eff;
  std::vector<int32_t> eff_start((size_t)n), eff_len((size_t)n);
  for (int k = 0; k < n; ++k) {
    eff_start[k] = (int32_t)eff.size();
    if (absorbed[k]) {
      const int p = s.par[k];
      const int32_t ps0 = eff_start[p], pl = eff_len[p];
      for (int32_t i = 0; i < pl; ++i) eff.push_back(eff[ps0 + i]);
    }
    eff.insert(eff.end(), s.pages.begin() + s.pg_off[k], s.pages.begin() + s.pg_off[k] + s.npages[k]);
    eff_len[k] = (int32_t)eff.size() - eff_start[k];
  }
  // each candidate's passes: (level, segment), levels in path order
  std::vector<int32_t> pass_off((size_t)num_cands + 1, 0), pass_seg;
  int num_levels = 0;
  for (int c = 0; c < num_cands; ++c) {
    for (int j = s.path_off[c]; j < s.path_off[c + 1]; ++j)
      if (!(j + 1 < s.path_off[c + 1] && absorbed[s.path[j + 1]])) pass_seg.push_back(s.path[j]);
    pass_off[c + 1] = (int32_t)pass_seg.size();
    num_levels = std::max(num_levels, pass_off[c + 1] - pass_off[c]);
  }
  const int L = num_cands > 0 ? num_levels : 0;
  buf.assign(2 + 5 * (size_t)L, 0);
  buf[0] = L;
  std::vector<int32_t> qo, kvp, kvi, lpl;
  for (int lv = 0; lv < L; ++lv) {
    qo.assign(1, 0), kvp.assign(1, 0), kvi.clear(), lpl.clear();
    int run_start = -1, run_prev = -1, run_key = -1;
    auto close_run = [&]() {
      if (run_start < 0) return;
      if (run_start > qo.back()) {                // candidates without a pass here
        qo.push_back(run_start);
        kvp.push_back((int32_t)kvi.size());
        lpl.push_back(0);
      }
      const int k = run_key;
      kvi.insert(kvi.end(), eff.begin() + eff_start[k], eff.begin() + eff_start[k] + eff_len[k]);
      kvp.push_back((int32_t)kvi.size());
      lpl.push_back(s.tokens[k] - (s.npages[k] - 1) * page_size);
      qo.push_back(run_prev + 1);
    };
    for (int c = 0; c < num_cands; ++c) {
      if (pass_off[c] + lv >= pass_off[c + 1]) continue;
      const int k = pass_seg[pass_off[c] + lv];
      if (run_start >= 0 && k == run_key && c == run_prev + 1) {
        run_prev = c;
        continue;
      }
      close_run();
      run_start = run_prev = c, run_key = k;
    }
    close_run();
    if (qo.back() < num_cands) {
      qo.push_back(num_cands);
      kvp.push_back((int32_t)kvi.size());
      lpl.push_back(0);
    }
    const int ng = (int)lpl.size();
    int32_t* hdr = buf.data() + 2 + 5 * lv;
    hdr[0] = ng;
    hdr[1] = (int32_t)buf.size();
    buf.insert(buf.end(), qo.begin(), qo.end());
    buf[2 + 5 * lv + 2] = (int32_t)buf.size();
    buf.insert(buf.end(), kvp.begin(), kvp.end());
    buf[2 + 5 * lv + 3] = (int32_t)buf.size();
    buf.insert(buf.end(), kvi.begin(), kvi.end());
    buf[2 + 5 * lv + 4] = (int32_t)buf.size();
    buf.insert(buf.end(), lpl.begin(), lpl.end());
  }
  return BE_OK;
}

}  // namespace

extern "C" int be_trie_cascade(const int32_t* parent, const int32_t* page, const int32_t* ntok,
                               const int32_t* last_tok, const uint8_t* alive, int num_nodes, const int32_t* leaves,
                               int num_cands, int32_t* out, int64_t out_capacity, int64_t* out_used) {
  if (out_used) *out_used = 0;
  int rc = check_inputs(parent, page, ntok, last_tok, alive, num_nodes, leaves, num_cands, out, out_capacity);
  if (rc != BE_OK) return rc;
  TrieWalk w;
  if ((rc = w.run(parent, page, ntok, alive, num_nodes)) != BE_OK) return rc;
  int max_level = 0;
  for (int c = 0; c < num_cands; ++c) max_level = std::max(max_level, w.lvl[leaves[c]]);
  const int L = num_cands > 0 ? max_level + 1 : 0;

  // key node of every (candidate, level): keys[c * L + lv]
  std::vector<int32_t> keys((size_t)num_cands * L);
  for (int c = 0; c < num_cands; ++c) {
    const int f = leaves[c];
    int32_t* k = keys.data() + (size_t)c * L;
    for (int lv = w.lvl[f]; lv < L; ++lv) k[lv] = f;
    int x = f;
    for (int lv = w.lvl[f] - 1; lv >= 0; --lv) {
      x = w.bp[x];
      k[lv] = x;
    }
  }

  // output: header [num_levels, off_cand], per level [groups, off_qo, off_kvp,
  // off_kvi, off_lpl], the level arrays, then the candidate block (query
  // token, write page, write slot, position; num_cands each)
  std::vector<int32_t> buf;
  buf.reserve(16 + 5 * (size_t)L + 8 * (size_t)num_cands * (L + 1));
  buf.resize(2 + 5 * (size_t)L, 0);
  std::vector<int32_t> gid((size_t)num_nodes, -1);
  std::vector<int32_t> seen((size_t)w.max_page + 1, -1);   // last group that listed the page
  int stamp = 0;
  std::vector<int32_t> gkey, gcount, glast, chain, kvi;
  for (int lv = 0; lv < L; ++lv) {
    gkey.clear(), gcount.clear(), glast.clear();
    for (int c = 0; c < num_cands; ++c) {
      const int k = keys[(size_t)c * L + lv];
      if (gid[k] < 0) {
        gid[k] = (int32_t)gkey.size();
        gkey.push_back(k);
        gcount.push_back(0);
        glast.push_back(k == leaves[c] ? std::max(0, ntok[k] - 1) : ntok[k]);
      }
      gcount[gid[k]] += 1;
    }
    const int ng = (int)gkey.size();
    int32_t* hdr = buf.data() + 2 + 5 * lv;
    hdr[0] = ng;
    hdr[1] = (int32_t)buf.size();
    buf.push_back(0);
    for (int i = 0; i < ng; ++i) buf.push_back(buf.back() + gcount[i]);
    buf[2 + 5 * lv + 2] = (int32_t)buf.size();
    const size_t kvp0 = buf.size();
    buf.resize(kvp0 + ng + 1, 0);
    kvi.clear();
    for (int i = 0; i < ng; ++i) {
      chain_pages(w, parent, page, gkey[i], chain, seen, stamp, kvi);
      buf[kvp0 + i + 1] = (int32_t)kvi.size();
    }
    buf[2 + 5 * lv + 3] = (int32_t)buf.size();
    buf.insert(buf.end(), kvi.begin(), kvi.end());
    buf[2 + 5 * lv + 4] = (int32_t)buf.size();
    buf.insert(buf.end(), glast.begin(), glast.end());
    for (int k : gkey) gid[k] = -1;
  }
  buf[0] = L;
  return finish(buf, w, page, ntok, last_tok, leaves, num_cands, out, out_capacity, out_used);
}

extern "C" int be_trie_levels(const int32_t* parent, const int32_t* page, const int32_t* ntok,
                              const int32_t* last_tok, const uint8_t* alive, int num_nodes, const int32_t* leaves,
                              int num_cands, int page_size, int kind, int include_self, const be_tree_model* model,
                              int32_t* out, int64_t out_capacity, int64_t* out_used, int32_t* chosen,
                              double* option_costs) {
  using be::fail;
  if (out_used) *out_used = 0;
  if (kind == BE_KIND_CASCADE) {
    if (include_self) return fail(BE_ERR_UNSUPPORTED, "the cascade levels exclude each candidate's newest token");
    if (chosen) *chosen = BE_KIND_CASCADE;
    return be_trie_cascade(parent, page, ntok, last_tok, alive, num_nodes, leaves, num_cands, out, out_capacity,
                           out_used);
  }
  if (kind < BE_KIND_FLAT || kind > BE_KIND_AUTO) return fail(BE_ERR_INVALID, "unknown strategy kind %d", kind);
  if (page_size <= 0) return fail(BE_ERR_INVALID, "page_size must be positive");
  const bool priced = kind == BE_KIND_TREE || kind == BE_KIND_AUTO;
  Costs cm{model, 1, 1, false};
  if (priced) {
    if (!model) return fail(BE_ERR_INVALID, "strategy kind %d needs a cost model", kind);
    if (model->num_kv_heads <= 0 || model->num_qo_heads <= 0 || model->num_qo_heads % model->num_kv_heads)
      return fail(BE_ERR_INVALID, "cost model heads %d / %d", model->num_qo_heads, model->num_kv_heads);
    cm.hkv = model->num_kv_heads;
    cm.g = model->num_qo_heads / model->num_kv_heads;
    cm.tail_ok = page_size % 16 == 0 && cm.g <= 16;
    if (model->edge_model != BE_EDGES_FITTED && model->edge_model != BE_EDGES_FASTTREE)
      return fail(BE_ERR_INVALID, "unknown edge model %d", model->edge_model);
    if (model->edge_model == BE_EDGES_FASTTREE && cm.g > 16)
      return fail(BE_ERR_UNSUPPORTED, "FastTree's query tiles need a GQA group of at most 16 (got %d)", cm.g);
  }
  int rc = check_inputs(parent, page, ntok, last_tok, alive, num_nodes, leaves, num_cands, out, out_capacity);
  if (rc != BE_OK) return rc;
  TrieWalk w;
  if ((rc = w.run(parent, page, ntok, alive, num_nodes)) != BE_OK) return rc;
  SegTree s;
  build_segments(w, parent, page, ntok, leaves, num_cands, num_nodes, page_size, include_self != 0, s);
  const int n = s.size();

  std::vector<uint8_t> absorbed((size_t)n, 0);
  int use = kind;
  if (kind == BE_KIND_FLAT) {
    for (int k = 0; k < n; ++k) absorbed[k] = s.par[k] >= 0;
  } else if (kind == BE_KIND_TREE) {
    std::vector<int64_t> teff;
    absorb_edges(s, cm, absorbed, teff);
  } else if (kind == BE_KIND_AUTO) {
    // flat, split and tree priced with the fitted costs (the tree's edges by
    // the model asked for); the first of the cheapest is built
    const double c_flat = flat_cost(s, cm, num_cands);
    std::vector<uint8_t> none((size_t)n, 0);
    std::vector<int64_t> own(s.tokens.begin(), s.tokens.end());
    const double c_split = decomposition_cost(s, cm, none, own, num_cands);
    std::vector<uint8_t> tree_abs;
    std::vector<int64_t> teff;
    absorb_edges(s, cm, tree_abs, teff);
    be_tree_model fitted = *model;
    fitted.edge_model = BE_EDGES_FITTED;
    const Costs price{&fitted, cm.g, cm.hkv, cm.tail_ok};
    const double c_tree = decomposition_cost(s, price, tree_abs, teff, num_cands);
    if (option_costs) option_costs[0] = c_flat, option_costs[1] = c_split, option_costs[2] = c_tree;
    use = BE_KIND_FLAT;
    double best = c_flat;
    if (c_split < best) use = BE_KIND_SPLIT, best = c_split;
    if (c_tree < best) use = BE_KIND_TREE, best = c_tree;
    if (use == BE_KIND_FLAT)
      for (int k = 0; k < n; ++k) absorbed[k] = s.par[k] >= 0;
    else if (use == BE_KIND_TREE)
      absorbed = tree_abs;
  }
  if (chosen) *chosen = use;
  std::vector<int32_t> buf;
  emit_levels(s, absorbed, num_cands, page_size, buf);
  return finish(buf, w, page, ntok, last_tok, leaves, num_cands, out, out_capacity, out_used);
}

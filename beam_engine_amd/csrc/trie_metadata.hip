// Per-step cascade metadata of a live beam trie, on the host (no device code).
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

#include <vector>

#include "common.h"

extern "C" int be_trie_cascade(const int32_t* parent, const int32_t* page, const int32_t* ntok,
                               const int32_t* last_tok, const uint8_t* alive, int num_nodes, const int32_t* leaves,
                               int num_cands, int32_t* out, int64_t out_capacity, int64_t* out_used) {
  using be::fail;
  if (out_used) *out_used = 0;
  if (num_nodes < 0 || num_cands < 0) return fail(BE_ERR_INVALID, "negative node or candidate count");
  if (num_cands > 0 && (!parent || !page || !ntok || !last_tok || !alive || !leaves))
    return fail(BE_ERR_INVALID, "null node table or leaf list");
  if (!out && out_capacity > 0) return fail(BE_ERR_INVALID, "null output buffer");

  std::vector<int32_t> nchild((size_t)num_nodes, 0);
  for (int n = 0; n < num_nodes; ++n) {
    if (!alive[n]) continue;
    const int p = parent[n];
    if (p >= 0) {
      if (p >= n) return fail(BE_ERR_INVALID, "node %d: parent %d is not older than the node", n, p);
      if (!alive[p]) return fail(BE_ERR_INVALID, "node %d: parent %d is not live", n, p);
      nchild[p] += 1;
    }
  }
  // top-down pass: level, segment head, branch point closing the previous
  // level (the chain of these gives the lower levels' keys), tokens above
  std::vector<int32_t> lvl((size_t)num_nodes, 0), head((size_t)num_nodes, 0), bp((size_t)num_nodes, -1);
  std::vector<int64_t> pre((size_t)num_nodes, 0);
  for (int n = 0; n < num_nodes; ++n) {
    if (!alive[n]) continue;
    const int p = parent[n];
    if (p < 0) {
      lvl[n] = 0, head[n] = n, bp[n] = -1, pre[n] = 0;
    } else if (nchild[p] > 1) {
      lvl[n] = lvl[p] + 1, head[n] = n, bp[n] = p, pre[n] = pre[p] + ntok[p];
    } else {
      lvl[n] = lvl[p], head[n] = head[p], bp[n] = bp[p], pre[n] = pre[p] + ntok[p];
    }
  }
  int max_level = 0;
  for (int c = 0; c < num_cands; ++c) {
    const int f = leaves[c];
    if (f < 0 || f >= num_nodes || !alive[f]) return fail(BE_ERR_INVALID, "candidate %d: leaf %d is not live", c, f);
    max_level = std::max(max_level, lvl[f]);
  }
  const int L = num_cands > 0 ? max_level + 1 : 0;

  // key node of every (candidate, level): keys[c * L + lv]
  std::vector<int32_t> keys((size_t)num_cands * L);
  for (int c = 0; c < num_cands; ++c) {
    const int f = leaves[c];
    int32_t* k = keys.data() + (size_t)c * L;
    for (int lv = lvl[f]; lv < L; ++lv) k[lv] = f;
    int x = f;
    for (int lv = lvl[f] - 1; lv >= 0; --lv) {
      x = bp[x];
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
  int max_page = -1;
  for (int n = 0; n < num_nodes; ++n)
    if (alive[n]) {
      if (page[n] < 0) return fail(BE_ERR_INVALID, "node %d: negative page id", n);
      max_page = std::max(max_page, page[n]);
    }
  std::vector<int32_t> seen((size_t)max_page + 1, -1);   // last group that listed the page
  int stamp = 0;
  std::vector<int32_t> gkey, gcount, glast, chain;
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
    std::vector<int32_t> kvi;
    for (int i = 0; i < ng; ++i) {
      chain.clear();
      for (int x = gkey[i];; x = parent[x]) {
        chain.push_back(page[x]);
        if (x == head[gkey[i]]) break;
      }
      // path order; a page id repeated along the chain is kept once (first occurrence)
      ++stamp;
      for (size_t a = chain.size(); a-- > 0;) {
        if (seen[chain[a]] == stamp) continue;
        seen[chain[a]] = stamp;
        kvi.push_back(chain[a]);
      }
      buf[kvp0 + i + 1] = (int32_t)kvi.size();
    }
    buf[2 + 5 * lv + 3] = (int32_t)buf.size();
    buf.insert(buf.end(), kvi.begin(), kvi.end());
    buf[2 + 5 * lv + 4] = (int32_t)buf.size();
    buf.insert(buf.end(), glast.begin(), glast.end());
    for (int k : gkey) gid[k] = -1;
  }
  buf[0] = L;
  buf[1] = (int32_t)buf.size();
  for (int c = 0; c < num_cands; ++c) buf.push_back(ntok[leaves[c]] > 0 ? last_tok[leaves[c]] : 0);
  for (int c = 0; c < num_cands; ++c) buf.push_back(page[leaves[c]]);
  for (int c = 0; c < num_cands; ++c) buf.push_back(ntok[leaves[c]] - 1);
  for (int c = 0; c < num_cands; ++c) {
    const int64_t pos = pre[leaves[c]] + ntok[leaves[c]] - 1;
    if (pos > INT32_MAX) return fail(BE_ERR_INVALID, "candidate %d: position %lld overflows int32", c, (long long)pos);
    buf.push_back((int32_t)pos);
  }

  if (out_used) *out_used = (int64_t)buf.size();
  if ((int64_t)buf.size() > out_capacity)
    return fail(BE_ERR_CAPACITY, "cascade metadata needs %lld int32 words, buffer holds %lld",
                (long long)buf.size(), (long long)out_capacity);
  memcpy(out, buf.data(), buf.size() * sizeof(int32_t));
  return BE_OK;
}

// Native beam trie and page allocator for the decode loop (host only, no
// device code).
//
// The reference keeps its beam trie as Python objects and updates it after
// every selection (src/beam_engine/beam_state.py:101-209,
// add_filtered_results), allocating and freeing pages through its PageTable
// (src/beam_engine/page_table.py:77-124).  Here both live in C++ so that a
// decode step's bookkeeping -- prune, expand, fork copies, the next step's
// cascade metadata -- is one call instead of per-candidate Python work while
// the GPU waits:
//
//  * be_page_pool: the FIFO free list (a ring: oldest free page first, freed
//    pages to the back) with a reference count per page.  With one holder
//    per page this is exactly the reference's allocate / free behaviour, so
//    page ids come out in the reference's order.
//  * be_beam_trie: a node table in creation order (parent, page, token count,
//    tokens, live children, alive) and the live candidates (leaf node,
//    request, score).  be_trie_apply takes a step's selection in emission
//    order -- (parent candidate, token, score) entries, children of a
//    candidate in their selection order -- and applies the reference's rules:
//    every candidate without children is pruned first (its leaf and each
//    ancestor left childless free their pages, leaf upward, candidates in
//    order); then, candidates in order, a single child appends to a non-full
//    page or opens a new page, several children of a full page open a page
//    each, and several children of a partial page get a copy of it each
//    after the first (siblings under the same parent, listed before the
//    candidate), whose copies are returned for one device launch, before the
//    first child appends to the original page.  A child whose token is the
//    end-of-sequence id (when one is given) finishes its beam instead, with
//    its whole sequence kept.
//    A selection whose expansion needs more pages than the pool holds after
//    the prune fails (BE_ERR_CAPACITY) before the trie or the pool changes.
//  * be_trie_metadata: the cascade arrays and per-candidate inputs of the
//    live trie (be_trie_cascade over the node table); be_trie_plan /
//    be_trie_plan_kind: a strategy's levels (be_trie_levels) and their
//    attention plan in one call.

#include <cstring>
#include <new>
#include <vector>

#include "common.h"

struct be_page_pool {
  int num_pages = 0;
  std::vector<int32_t> ring;        // free list: ring[(head + i) % n], i < count, oldest first
  int head = 0, count = 0;
  std::vector<int32_t> refs;        // holders per page (0: free)

  bool take(int32_t& page) {
    if (count == 0) return false;
    page = ring[head];
    head = head + 1 == num_pages ? 0 : head + 1;
    --count;
    refs[page] = 1;
    return true;
  }
  void push_back(int32_t page) {
    int at = head + count;
    if (at >= num_pages) at -= num_pages;
    ring[at] = page;
    ++count;
  }
  // 1: the page went back to the free list, 0: still held, -1: not allocated
  int release(int32_t page) {
    if (page < 0 || page >= num_pages || refs[page] == 0) return -1;
    if (--refs[page] > 0) return 0;
    push_back(page);
    return 1;
  }
};

struct be_beam_trie {
  int page_size = 0;
  be_page_pool* pool = nullptr;
  // node table, creation order
  std::vector<int32_t> parent, page, ntok, last, nchild, tokens;   // tokens: page_size per node
  std::vector<uint8_t> alive;
  // live candidates
  std::vector<int32_t> cand_node, cand_req;
  std::vector<double> cand_score;
  // finished candidates (end-of-sequence picks)
  std::vector<int32_t> fin_req, fin_off;                           // fin_off: num_finished + 1 offsets
  std::vector<double> fin_score;
  std::vector<int32_t> fin_tokens;
  int64_t version = 0;                                             // bumped by every change

  int add_node(int32_t par, int32_t pg, const int32_t* toks, int n) {
    const int id = (int)parent.size();
    parent.push_back(par);
    page.push_back(pg);
    ntok.push_back(n);
    last.push_back(n > 0 ? toks[n - 1] : 0);
    nchild.push_back(0);
    alive.push_back(1);
    tokens.resize(tokens.size() + (size_t)page_size, 0);
    if (n > 0) std::memcpy(&tokens[(size_t)id * page_size], toks, sizeof(int32_t) * (size_t)n);
    if (par >= 0) nchild[par] += 1;
    return id;
  }
  void append_token(int node, int32_t tok) {
    tokens[(size_t)node * page_size + ntok[node]] = tok;
    ntok[node] += 1;
    last[node] = tok;
  }
  // Drop dead nodes, keeping the live ones in creation order (parents stay
  // below their children), once they are most of the table.
  void compact() {
    const int n = (int)parent.size();
    int live = 0;
    for (int i = 0; i < n; ++i) live += alive[i];
    if (n < 1024 || 2 * live > n) return;
    std::vector<int32_t> map((size_t)n, -1);
    int k = 0;
    for (int i = 0; i < n; ++i) {
      if (!alive[i]) continue;
      map[i] = k;
      parent[k] = parent[i] >= 0 ? map[parent[i]] : -1;
      page[k] = page[i];
      ntok[k] = ntok[i];
      last[k] = last[i];
      nchild[k] = nchild[i];
      alive[k] = 1;
      if (k != i)
        std::memmove(&tokens[(size_t)k * page_size], &tokens[(size_t)i * page_size], sizeof(int32_t) * page_size);
      ++k;
    }
    parent.resize(k), page.resize(k), ntok.resize(k), last.resize(k), nchild.resize(k), alive.resize(k);
    tokens.resize((size_t)k * page_size);
    for (auto& c : cand_node) c = map[c];
  }
  void sequence(int node, std::vector<int32_t>& out) const {
    std::vector<int> path;
    for (int n = node; n >= 0; n = parent[n]) path.push_back(n);
    for (size_t i = path.size(); i-- > 0;) {
      const int n = path[i];
      out.insert(out.end(), &tokens[(size_t)n * page_size], &tokens[(size_t)n * page_size] + ntok[n]);
    }
  }
};

extern "C" {

// ---------------------------------------------------------------- page pool
be_page_pool* be_pages_create(int num_pages) {
  if (num_pages <= 0) {
    be::fail(BE_ERR_INVALID, "num_pages must be positive");
    return nullptr;
  }
  be_page_pool* p = new (std::nothrow) be_page_pool();
  if (!p) {
    be::fail(BE_ERR_CAPACITY, "out of host memory");
    return nullptr;
  }
  p->num_pages = num_pages;
  p->ring.resize((size_t)num_pages);
  p->refs.assign((size_t)num_pages, 0);
  for (int i = 0; i < num_pages; ++i) p->ring[i] = i;
  p->count = num_pages;
  return p;
}

void be_pages_destroy(be_page_pool* p) { delete p; }

int be_pages_allocate(be_page_pool* p, int32_t* page) {
  BE_REQUIRE(p && page, "null pool or output");
  if (!p->take(*page)) return be::fail(BE_ERR_CAPACITY, "No free pages available");
  return BE_OK;
}

int be_pages_share(be_page_pool* p, int page, int32_t* count) {
  BE_REQUIRE(p, "null pool");
  if (page < 0 || page >= p->num_pages || p->refs[page] == 0)
    return be::fail(BE_ERR_INVALID, "Page %d is not allocated", page);
  p->refs[page] += 1;
  if (count) *count = p->refs[page];
  return BE_OK;
}

int be_pages_release(be_page_pool* p, int page, int32_t* state) {
  BE_REQUIRE(p, "null pool");
  const int s = p->release(page);
  if (state) *state = s;
  return BE_OK;
}

int be_pages_reserve(be_page_pool* p, int page) {
  BE_REQUIRE(p, "null pool");
  if (page < 0 || page >= p->num_pages) return be::fail(BE_ERR_INVALID, "page %d outside the pool", page);
  if (p->refs[page] != 0) return be::fail(BE_ERR_INVALID, "Page %d is already allocated", page);
  // take it out of the ring, keeping the order of the others
  int at = -1;
  for (int i = 0; i < p->count; ++i) {
    int j = p->head + i;
    if (j >= p->num_pages) j -= p->num_pages;
    if (p->ring[j] == page) {
      at = i;
      break;
    }
  }
  if (at < 0) return be::fail(BE_ERR_INVALID, "page %d is not in the free list", page);
  for (int i = at; i + 1 < p->count; ++i) {
    int j = p->head + i, k = j + 1;
    if (j >= p->num_pages) j -= p->num_pages;
    if (k >= p->num_pages) k -= p->num_pages;
    p->ring[j] = p->ring[k];
  }
  p->count -= 1;
  p->refs[page] = 1;
  return BE_OK;
}

int be_pages_num_free(const be_page_pool* p) { return p ? p->count : 0; }

int be_pages_ref_count(const be_page_pool* p, int page) {
  if (!p || page < 0 || page >= p->num_pages) return 0;
  return p->refs[page];
}

int be_pages_free_list(const be_page_pool* p, int32_t* out, int cap) {
  if (!p) return 0;
  const int n = p->count < cap ? p->count : cap;
  for (int i = 0; i < n; ++i) {
    int j = p->head + i;
    if (j >= p->num_pages) j -= p->num_pages;
    out[i] = p->ring[j];
  }
  return p->count;
}

// ---------------------------------------------------------------- trie
be_beam_trie* be_trie_create(int page_size, be_page_pool* pool) {
  if (page_size <= 0 || !pool) {
    be::fail(BE_ERR_INVALID, "page_size must be positive and the pool non-null");
    return nullptr;
  }
  be_beam_trie* t = new (std::nothrow) be_beam_trie();
  if (!t) {
    be::fail(BE_ERR_CAPACITY, "out of host memory");
    return nullptr;
  }
  t->page_size = page_size;
  t->pool = pool;
  t->fin_off.push_back(0);
  return t;
}

void be_trie_destroy(be_beam_trie* t) { delete t; }

int be_trie_add_root(be_beam_trie* t, const int32_t* tokens, int n, int request_id, int32_t* pages_out) {
  BE_REQUIRE(t && (tokens || n == 0), "null trie or tokens");
  BE_REQUIRE(n > 0, "a root sequence needs at least one token");
  const int ps = t->page_size;
  int cur = -1, k = 0;
  for (int s = 0; s < n; s += ps) {
    int32_t pg;
    if (!t->pool->take(pg)) return be::fail(BE_ERR_CAPACITY, "No free pages available");
    const int len = n - s < ps ? n - s : ps;
    cur = t->add_node(cur, pg, tokens + s, len);
    if (pages_out) pages_out[k] = pg;
    ++k;
  }
  t->cand_node.push_back(cur);
  t->cand_req.push_back(request_id);
  t->cand_score.push_back(0.0);
  t->version += 1;
  return BE_OK;
}

int be_trie_apply(be_beam_trie* t, const int32_t* sel_parent, const int32_t* sel_token, const double* sel_score,
                  int n_entries, int eos_token, int32_t* copies, int copies_cap, int* n_copies,
                  int* n_release_warnings) {
  BE_REQUIRE(t, "null trie");
  BE_REQUIRE(n_entries >= 0 && (n_entries == 0 || (sel_parent && sel_token && sel_score)), "null selection");
  BE_REQUIRE(n_copies, "null copy count");
  // every copy is one child's: room for one per entry means room for all
  BE_REQUIRE(copies && copies_cap >= n_entries, "copy list needs room for %d entries", n_entries);
  const int nc = (int)t->cand_node.size();
  const int ps = t->page_size;
  // children of each candidate, in entry order
  std::vector<int> cnt((size_t)nc + 1, 0);
  for (int e = 0; e < n_entries; ++e) {
    const int p = sel_parent[e];
    if (p < 0) continue;
    if (p >= nc) return be::fail(BE_ERR_INVALID, "selection entry %d names candidate %d of %d", e, p, nc);
    cnt[p + 1] += 1;
  }
  for (int i = 0; i < nc; ++i) cnt[i + 1] += cnt[i];
  std::vector<int> kids((size_t)cnt[nc]);
  {
    std::vector<int> at(cnt.begin(), cnt.end() - 1);
    for (int e = 0; e < n_entries; ++e)
      if (sel_parent[e] >= 0) kids[at[sel_parent[e]]++] = e;
  }
  // end-of-sequence picks finish their beams (the other children go on)
  std::vector<int> live_cnt((size_t)nc, 0);
  for (int i = 0; i < nc; ++i)
    for (int q = cnt[i]; q < cnt[i + 1]; ++q)
      if (!(eos_token >= 0 && sel_token[kids[q]] == eos_token)) live_cnt[i] += 1;
  // The pages the expansion takes (a single child on a full page: one; m
  // children on a full page: m; on a partial page: m - 1 copies) against the
  // free list after the prune (pages whose last holder the prune releases,
  // found on a copy of the child counts): a selection the pool cannot hold
  // fails here, before anything changes.
  {
    int64_t need = 0;
    for (int i = 0; i < nc; ++i) {
      const int m = live_cnt[i];
      if (m == 0) continue;
      const int node = t->cand_node[i];
      need += m == 1 ? (t->ntok[node] < ps ? 0 : 1) : (t->ntok[node] == ps ? m : m - 1);
    }
    int64_t avail = t->pool->count;
    if (need > avail) {
      std::vector<int32_t> kc(t->nchild);
      std::vector<uint8_t> gone(t->alive.size(), 0);
      for (int i = 0; i < nc && need > avail; ++i) {
        if (live_cnt[i] > 0) continue;
        int node = t->cand_node[i];
        while (node >= 0 && t->alive[node] && !gone[node] && kc[node] == 0) {
          gone[node] = 1;
          const int32_t pg = t->page[node];
          if (pg >= 0 && pg < t->pool->num_pages && t->pool->refs[pg] == 1) ++avail;
          const int par = t->parent[node];
          if (par >= 0) kc[par] -= 1;
          node = par;
        }
      }
    }
    if (need > avail)
      return be::fail(BE_ERR_CAPACITY, "No free pages available (the step needs %lld, %lld free after pruning)",
                      (long long)need, (long long)avail);
  }
  for (int i = 0; i < nc; ++i)
    for (int q = cnt[i]; q < cnt[i + 1]; ++q) {
      const int e = kids[q];
      if (eos_token >= 0 && sel_token[e] == eos_token) {
        t->fin_req.push_back(t->cand_req[i]);
        t->fin_score.push_back(sel_score[e]);
        t->sequence(t->cand_node[i], t->fin_tokens);
        t->fin_tokens.push_back(sel_token[e]);
        t->fin_off.push_back((int32_t)t->fin_tokens.size());
        kids[q] = -1;
      }
    }
  // prune: leaf upward while childless, candidates in order
  int warnings = 0;
  for (int i = 0; i < nc; ++i) {
    if (live_cnt[i] > 0) continue;
    int node = t->cand_node[i];
    while (node >= 0 && t->alive[node] && t->nchild[node] == 0) {
      if (t->pool->release(t->page[node]) < 0) ++warnings;
      t->alive[node] = 0;
      const int par = t->parent[node];
      if (par >= 0) t->nchild[par] -= 1;
      node = par;
    }
  }
  t->version += 1;                 // the state has changed from here on
  // expand, candidates in order
  std::vector<int32_t> nn, nr;
  std::vector<double> nsc;
  nn.reserve((size_t)n_entries);
  nr.reserve((size_t)n_entries);
  nsc.reserve((size_t)n_entries);
  int ncp = 0;
  std::vector<int32_t> buf((size_t)ps + 1);
  for (int i = 0; i < nc; ++i) {
    if (live_cnt[i] == 0) continue;
    std::vector<int> lk;
    lk.reserve((size_t)live_cnt[i]);
    for (int q = cnt[i]; q < cnt[i + 1]; ++q)
      if (kids[q] >= 0) lk.push_back(kids[q]);
    const int node = t->cand_node[i], rid = t->cand_req[i];
    if (lk.size() == 1) {
      const int e = lk[0];
      if (t->ntok[node] < ps) {
        t->append_token(node, sel_token[e]);
        nn.push_back(node);
      } else {
        int32_t pg;
        if (!t->pool->take(pg)) return be::fail(BE_ERR_CAPACITY, "No free pages available");
        nn.push_back(t->add_node(node, pg, &sel_token[e], 1));
      }
      nr.push_back(rid);
      nsc.push_back(sel_score[e]);
      continue;
    }
    if (t->ntok[node] == ps) {
      for (int e : lk) {
        int32_t pg;
        if (!t->pool->take(pg)) return be::fail(BE_ERR_CAPACITY, "No free pages available");
        nn.push_back(t->add_node(node, pg, &sel_token[e], 1));
        nr.push_back(rid);
        nsc.push_back(sel_score[e]);
      }
      continue;
    }
    const int len = t->ntok[node];
    for (size_t q = 1; q < lk.size(); ++q) {
      const int e = lk[q];
      int32_t pg;
      if (!t->pool->take(pg)) return be::fail(BE_ERR_CAPACITY, "No free pages available");
      copies[3 * ncp + 0] = t->page[node];
      copies[3 * ncp + 1] = pg;
      copies[3 * ncp + 2] = len;
      ++ncp;
      std::memcpy(buf.data(), &t->tokens[(size_t)node * ps], sizeof(int32_t) * (size_t)len);
      buf[len] = sel_token[e];
      nn.push_back(t->add_node(t->parent[node], pg, buf.data(), len + 1));
      nr.push_back(rid);
      nsc.push_back(sel_score[e]);
    }
    t->append_token(node, sel_token[lk[0]]);
    nn.push_back(node);
    nr.push_back(rid);
    nsc.push_back(sel_score[lk[0]]);
  }
  t->cand_node.swap(nn);
  t->cand_req.swap(nr);
  t->cand_score.swap(nsc);
  t->compact();
  t->version += 1;
  *n_copies = ncp;
  if (n_release_warnings) *n_release_warnings = warnings;
  return BE_OK;
}

// Sizes of the state: [nodes, candidates, finished, finished tokens, page_size], and the version.
int be_trie_sizes(const be_beam_trie* t, int32_t* out5, int64_t* version) {
  BE_REQUIRE(t && out5, "null trie or output");
  out5[0] = (int32_t)t->parent.size();
  out5[1] = (int32_t)t->cand_node.size();
  out5[2] = (int32_t)t->fin_req.size();
  out5[3] = (int32_t)t->fin_tokens.size();
  out5[4] = t->page_size;
  if (version) *version = t->version;
  return BE_OK;
}

// The live candidates: leaf node, request, score (num_candidates each).
int be_trie_candidates(const be_beam_trie* t, int32_t* node, int32_t* request, double* score) {
  BE_REQUIRE(t, "null trie");
  const size_t n = t->cand_node.size();
  if (node) std::memcpy(node, t->cand_node.data(), n * sizeof(int32_t));
  if (request) std::memcpy(request, t->cand_req.data(), n * sizeof(int32_t));
  if (score) std::memcpy(score, t->cand_score.data(), n * sizeof(double));
  return BE_OK;
}

// The node table (num_nodes rows; tokens: page_size per node) and the
// finished candidates (request, score, token offsets num_finished + 1, tokens).
int be_trie_export(const be_beam_trie* t, int32_t* parent, int32_t* page, int32_t* ntok, uint8_t* alive,
                   int32_t* tokens, int32_t* fin_req, double* fin_score, int32_t* fin_off, int32_t* fin_tokens) {
  BE_REQUIRE(t, "null trie");
  const size_t n = t->parent.size();
  if (parent) std::memcpy(parent, t->parent.data(), n * sizeof(int32_t));
  if (page) std::memcpy(page, t->page.data(), n * sizeof(int32_t));
  if (ntok) std::memcpy(ntok, t->ntok.data(), n * sizeof(int32_t));
  if (alive) std::memcpy(alive, t->alive.data(), n);
  if (tokens) std::memcpy(tokens, t->tokens.data(), t->tokens.size() * sizeof(int32_t));
  const size_t f = t->fin_req.size();
  if (fin_req) std::memcpy(fin_req, t->fin_req.data(), f * sizeof(int32_t));
  if (fin_score) std::memcpy(fin_score, t->fin_score.data(), f * sizeof(double));
  if (fin_off) std::memcpy(fin_off, t->fin_off.data(), (f + 1) * sizeof(int32_t));
  if (fin_tokens) std::memcpy(fin_tokens, t->fin_tokens.data(), t->fin_tokens.size() * sizeof(int32_t));
  return BE_OK;
}

// The cascade metadata of the live trie, as be_trie_cascade lays it out.
int be_trie_metadata(const be_beam_trie* t, int32_t* out, int64_t out_capacity, int64_t* out_used) {
  BE_REQUIRE(t, "null trie");
  return be_trie_cascade(t->parent.data(), t->page.data(), t->ntok.data(), t->last.data(), t->alive.data(),
                         (int)t->parent.size(), t->cand_node.data(), (int)t->cand_node.size(), out, out_capacity,
                         out_used);
}

// One strategy's levels of the live trie, as be_trie_levels lays them out.
int be_trie_metadata_kind(const be_beam_trie* t, int kind, int include_self, const be_tree_model* model, int32_t* out,
                          int64_t out_capacity, int64_t* out_used, int32_t* chosen, double* option_costs) {
  BE_REQUIRE(t, "null trie");
  return be_trie_levels(t->parent.data(), t->page.data(), t->ntok.data(), t->last.data(), t->alive.data(),
                        (int)t->parent.size(), t->cand_node.data(), (int)t->cand_node.size(), t->page_size, kind,
                        include_self, model, out, out_capacity, out_used, chosen, option_costs);
}

// The step's metadata (into meta, as be_trie_metadata) and the cascade
// attention plan of its levels (be_attn_plan into host_plan): the per-step
// host work of a cascade decode step in one call.  The last level's groups
// get the causal mask when one holds more than one query (as the cascade
// wrapper's plan decides it); *max_page is the largest page id the levels
// name (-1 for none).
int be_trie_plan(const be_beam_trie* t, int num_qo_heads, int num_kv_heads, int head_dim, int dtype, int flags,
                 int num_cus, const be_plan_caps* caps, int32_t* meta, int64_t meta_capacity, int64_t* meta_used,
                 int32_t* host_plan, int64_t host_plan_capacity, be_attn_plan_info* info, int32_t* max_page) {
  return be_trie_plan_kind(t, BE_KIND_CASCADE, 0, nullptr, num_qo_heads, num_kv_heads, head_dim, dtype, flags,
                           num_cus, caps, meta, meta_capacity, meta_used, host_plan, host_plan_capacity, info,
                           max_page, nullptr, nullptr);
}

// be_trie_plan for any strategy kind: the levels of be_trie_levels, then
// the attention plan of those levels.
int be_trie_plan_kind(const be_beam_trie* t, int kind, int include_self, const be_tree_model* model,
                      int num_qo_heads, int num_kv_heads, int head_dim, int dtype, int flags, int num_cus,
                      const be_plan_caps* caps, int32_t* meta, int64_t meta_capacity, int64_t* meta_used,
                      int32_t* host_plan, int64_t host_plan_capacity, be_attn_plan_info* info, int32_t* max_page,
                      int32_t* chosen, double* option_costs) {
  BE_REQUIRE(t && meta_used && info && max_page, "null argument");
  int32_t used_kind = kind;
  const int rc = be_trie_levels(t->parent.data(), t->page.data(), t->ntok.data(), t->last.data(), t->alive.data(),
                                (int)t->parent.size(), t->cand_node.data(), (int)t->cand_node.size(), t->page_size,
                                kind, include_self, model, meta, meta_capacity, meta_used, &used_kind, option_costs);
  if (chosen) *chosen = used_kind;
  if (rc != BE_OK) return rc;
  const int nl = meta[0];
  const int nc = (int)t->cand_node.size();
  std::vector<be_level> lv((size_t)(nl > 0 ? nl : 1));
  int32_t mp = -1;
  bool mask = false;
  for (int l = 0; l < nl; ++l) {
    const int32_t* rec = meta + 2 + 5 * l;
    const int ng = rec[0];
    lv[l] = be_level{meta + rec[1], meta + rec[2], meta + rec[3], meta + rec[4], ng};
    const int32_t* kvp = meta + rec[2];
    const int32_t* kvi = meta + rec[3];
    for (int32_t i = 0; i < kvp[ng]; ++i) mp = kvi[i] > mp ? kvi[i] : mp;
    if (l == nl - 1 && used_kind == BE_KIND_CASCADE)
      for (int gi = 0; gi < ng; ++gi)
        if (meta[rec[1] + gi + 1] - meta[rec[1] + gi] > 1) mask = true;
  }
  *max_page = mp;
  return be_attn_plan(lv.data(), nl, nc, num_qo_heads, num_kv_heads, head_dim, t->page_size, mp + 1 > 1 ? mp + 1 : 1,
                      dtype, flags | (mask ? BE_PLAN_CAUSAL : 0), num_cus, caps, host_plan, host_plan_capacity,
                      info);
}

}  // extern "C"

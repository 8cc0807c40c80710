"""CPU restatement of the reference's decode attention (test infrastructure).

Everything is computed in float64 with numpy, whatever the storage dtype of
the inputs.  Log-sum-exp values are natural logarithms, as in the reference's
FastTree kernels (attention/fasttree/kernel.py:92-93, 118, 243-245).

Semantics restated:

* paged gather -- a group with pages p0..p(n-1) and last-page length l covers
  every slot of p0..p(n-2) followed by slots 0..l-1 of p(n-1); K lives at
  ``kv[:, 0]`` and V at ``kv[:, 1]`` of the per-layer ``[P, 2, page, Hkv, D]``
  tensor (page_table.py:62-72; FlashInfer's kv_len rule as planned at
  models/modeling_llama.py:742-755).
* partial attention -- s_i = (q . k_i) * sm_scale, o = softmax(s) V,
  lse = m + ln sum exp(s - m); query head h reads KV head h // (Hq/Hkv)
  (attention/fasttree/kernel.py:34-119).  An empty KV set gives (0, -inf).
* merge -- o = sum_i e^(lse_i - M) o_i / sum_i e^(lse_i - M),
  lse = M + ln sum_i e^(lse_i - M) (attention/fasttree/kernel.py:188-252).
* cascade -- merge over levels of the partial attention of each query over
  its level group (MultiLevelCascadeAttentionWrapper.run as called at
  models/modeling_llama.py:321-367; index layout of cascade.md:34-54).
"""

from __future__ import annotations

import math
from typing import List, Sequence, Tuple

import numpy as np

NEG_INF = -math.inf


def _as_f64(x) -> np.ndarray:
    """Convert a numpy array or a (CPU) torch tensor to a float64 numpy array."""
    if hasattr(x, "detach"):
        x = x.detach().cpu()
        if str(x.dtype) in ("torch.bfloat16", "torch.float16"):
            x = x.float()
        x = x.numpy()
    return np.asarray(x, dtype=np.float64)


def group_slots(pages: Sequence[int], last_len: int, page_size: int) -> List[Tuple[int, int]]:
    """(page, slot) pairs a paged group covers, in order (Appendix-B.1 gather rule)."""
    pages = [int(p) for p in pages]
    out: List[Tuple[int, int]] = []
    for i, p in enumerate(pages):
        n = page_size if i + 1 < len(pages) else int(last_len)
        out.extend((p, s) for s in range(n))
    return out


def gather_kv(kv_layer, pages: Sequence[int], last_len: int, page_size: int):
    """K, V of one paged group as float64 arrays ``[T, Hkv, D]``.

    Follows the per-layer layout of page_table.py:62-72 (K at index 0, V at 1).
    """
    kv = _as_f64(kv_layer)
    slots = group_slots(pages, last_len, page_size)
    hkv, d = kv.shape[3], kv.shape[4]
    if not slots:
        z = np.zeros((0, hkv, d))
        return z, z.copy()
    pg = np.array([p for p, _ in slots])
    sl = np.array([s for _, s in slots])
    return kv[pg, 0, sl], kv[pg, 1, sl]


def partial_attention(q, k, v, sm_scale: float):
    """Softmax attention of queries ``q [n, Hq, D]`` over ``k, v [T, Hkv, D]``.

    Returns ``(o [n, Hq, D], lse [n, Hq])`` in float64, natural-log lse.
    Restates attention/fasttree/kernel.py:62-119 (online softmax, normalised
    output, lse = ln(sum) + max) in closed form.  T == 0 gives (0, -inf).
    """
    q = _as_f64(q)
    k = _as_f64(k)
    v = _as_f64(v)
    n, hq, d = q.shape
    t, hkv = k.shape[0], k.shape[1]
    o = np.zeros((n, hq, d))
    lse = np.full((n, hq), NEG_INF)
    if t == 0 or n == 0:
        return o, lse
    g = hq // hkv
    # head h reads kv head h // g  (kernel.py:46, cur_qo_head = cur_kv_head * g)
    kh = np.repeat(k, g, axis=1)  # [T, Hq, D]
    vh = np.repeat(v, g, axis=1)
    s = np.einsum("nhd,thd->nht", q, kh) * sm_scale
    m = s.max(axis=2, keepdims=True)
    p = np.exp(s - m)
    z = p.sum(axis=2, keepdims=True)
    o = np.einsum("nht,thd->nhd", p, vh) / z
    lse = (m + np.log(z))[..., 0]
    return o, lse


def merge_states(os_: Sequence[np.ndarray], lses: Sequence[np.ndarray]):
    """Log-sum-exp merge of partial states (attention/fasttree/kernel.py:210-252).

    ``os_[i]`` is ``[..., D]`` and ``lses[i]`` is ``[...]``.  Entries whose lse
    is -inf contribute nothing; if every entry is -inf the result is (0, -inf).
    """
    lse_stack = np.stack([_as_f64(x) for x in lses])          # [k, ...]
    o_stack = np.stack([_as_f64(x) for x in os_])              # [k, ..., D]
    finite = np.isfinite(lse_stack)
    m = np.where(finite, lse_stack, NEG_INF).max(axis=0)       # [...]
    m_safe = np.where(np.isfinite(m), m, 0.0)
    w = np.where(finite, np.exp(np.where(finite, lse_stack, 0.0) - m_safe), 0.0)
    z = w.sum(axis=0)
    z_safe = np.where(z > 0, z, 1.0)
    o = (w[..., None] * o_stack).sum(axis=0) / z_safe[..., None]
    o = np.where((z > 0)[..., None], o, 0.0)
    lse = np.where(z > 0, m_safe + np.log(z_safe), NEG_INF)
    return o, lse


def cascade_attention(q, kv_layer, qo_indptr_arr, kv_indptr_arr, kv_indices_arr,
                      last_page_len_arr, page_size: int, sm_scale: float | None = None, causal: bool = False):
    """Multi-level cascade decode attention, float64.

    For every level and every group gamma (queries qo_indptr[g]..qo_indptr[g+1],
    pages kv_indices[kv_indptr[g]:kv_indptr[g+1]], last length
    last_page_len[g]) computes the partial attention of the group's queries
    and merges the levels by log-sum-exp.  sm_scale defaults to D^-0.5
    (models/modeling_llama.py:304, 753).  Returns ``(o [N, Hq, D], lse [N, Hq])``.

    ``causal`` masks the last level's groups as FlashInfer's causal prefill
    does (the reference plans its prefill with causal=True,
    models/modeling_llama.py:775-798): query i of a group of n queries over T
    tokens sees the first T - n + i + 1 of them (the query block aligned to
    the end of the keys; n == T is the plain lower-triangular mask).
    """
    qf = _as_f64(q)
    n, hq, d = qf.shape
    if sm_scale is None:
        sm_scale = d ** -0.5
    level_o, level_lse = [], []
    n_levels = len(qo_indptr_arr)
    for li, (qo, kvp, kvi, lpl) in enumerate(zip(qo_indptr_arr, kv_indptr_arr, kv_indices_arr, last_page_len_arr)):
        qo = [int(x) for x in qo]
        kvp = [int(x) for x in kvp]
        kvi = [int(x) for x in kvi]
        lpl = [int(x) for x in lpl]
        o_l = np.zeros((n, hq, d))
        lse_l = np.full((n, hq), NEG_INF)
        for gi in range(len(qo) - 1):
            pages = kvi[kvp[gi]:kvp[gi + 1]]
            k, v = gather_kv(kv_layer, pages, lpl[gi] if pages else 0, page_size)
            nq = qo[gi + 1] - qo[gi]
            if causal and li == n_levels - 1 and nq > 1:
                t = k.shape[0]
                for i in range(nq):
                    vis = max(0, min(t, t - nq + i + 1))
                    o_g, lse_g = partial_attention(qf[qo[gi] + i:qo[gi] + i + 1], k[:vis], v[:vis], sm_scale)
                    o_l[qo[gi] + i] = o_g[0]
                    lse_l[qo[gi] + i] = lse_g[0]
                continue
            o_g, lse_g = partial_attention(qf[qo[gi]:qo[gi + 1]], k, v, sm_scale)
            o_l[qo[gi]:qo[gi + 1]] = o_g
            lse_l[qo[gi]:qo[gi + 1]] = lse_g
        level_o.append(o_l)
        level_lse.append(lse_l)
    return merge_states(level_o, level_lse)


def paged_attention(q, kv_layer, kv_indptr, kv_indices, last_page_len, page_size: int,
                    sm_scale: float | None = None):
    """Flat paged decode attention: query i attends to its own page list i."""
    n = _as_f64(q).shape[0]
    return cascade_attention(q, kv_layer, [list(range(n + 1))], [kv_indptr], [kv_indices],
                             [last_page_len], page_size, sm_scale)


def reference_attention_dense(q, k, v, sm_scale: float):
    """Dense float64 attention by explicit loops (tiny shapes only; pins partial_attention)."""
    q = _as_f64(q)
    k = _as_f64(k)
    v = _as_f64(v)
    n, hq, d = q.shape
    t, hkv = k.shape[0], k.shape[1]
    g = hq // hkv
    o = np.zeros((n, hq, d))
    lse = np.full((n, hq), NEG_INF)
    for i in range(n):
        for h in range(hq):
            if t == 0:
                continue
            s = [sum(q[i, h, e] * k[j, h // g, e] for e in range(d)) * sm_scale for j in range(t)]
            m = max(s)
            w = [math.exp(x - m) for x in s]
            z = sum(w)
            for e in range(d):
                o[i, h, e] = sum(w[j] * v[j, h // g, e] for j in range(t)) / z
            lse[i, h] = m + math.log(z)
    return o, lse


def cascade_attention_torch(q, kv_layer, qo_indptr_arr, kv_indptr_arr, kv_indices_arr, last_page_len_arr,
                            page_size: int, sm_scale: float | None = None):
    """The same multi-level cascade decode attention in torch float32 on the
    CPU -- the form the bench's CPU baseline times (paged gather, per-level softmax
    attention with (o, lse), log-sum-exp merge), using torch's threads.

    ``q [N, Hq, D]`` and ``kv_layer [P, 2, page, Hkv, D]`` are CPU tensors
    (any float dtype, computed in float32).  Returns ``(o, lse)`` float32
    tensors; pinned against ``cascade_attention`` (float64) in the tests."""
    import torch
    q = q.float()
    kv = kv_layer
    n, hq, d = q.shape
    hkv = kv.shape[3]
    g = hq // hkv
    if sm_scale is None:
        sm_scale = d ** -0.5
    o_acc = torch.zeros((n, hq, d), dtype=torch.float32)
    m_acc = torch.full((n, hq), NEG_INF, dtype=torch.float32)
    z_acc = torch.zeros((n, hq), dtype=torch.float32)
    slot_off = torch.arange(page_size)
    k_flat = kv[:, 0].reshape(-1, hkv, d)         # [P * page, Hkv, D] (a copy of the K half)
    v_flat = kv[:, 1].reshape(-1, hkv, d)
    for qo, kvp, kvi, lpl in zip(qo_indptr_arr, kv_indptr_arr, kv_indices_arr, last_page_len_arr):
        qo = [int(x) for x in qo]
        kvp = [int(x) for x in kvp]
        kvi_t = torch.as_tensor([int(x) for x in kvi], dtype=torch.long)
        for gi in range(len(qo) - 1):
            a, b = qo[gi], qo[gi + 1]
            pages = kvi_t[kvp[gi]:kvp[gi + 1]]
            if b <= a or pages.numel() == 0:
                continue
            t = (pages.numel() - 1) * page_size + int(lpl[gi])
            if t <= 0:
                continue
            flat = (pages[:, None] * page_size + slot_off[None, :]).reshape(-1)[:t]
            kk = k_flat.index_select(0, flat).float()                            # [T, Hkv, D]
            vv = v_flat.index_select(0, flat).float()
            qg = q[a:b].reshape(b - a, hkv, g, d).permute(1, 0, 2, 3).reshape(hkv, (b - a) * g, d)
            s = torch.bmm(qg, kk.permute(1, 2, 0).contiguous()) * sm_scale    # [Hkv, nq*g, T]
            m = s.amax(dim=2)
            p = torch.exp(s - m[..., None])
            z = p.sum(dim=2)
            og = torch.bmm(p, vv.permute(1, 0, 2).contiguous())                # [Hkv, nq*g, D] unnormalised
            og = og.reshape(hkv, b - a, g, d).permute(1, 0, 2, 3).reshape(b - a, hq, d)
            m = m.reshape(hkv, b - a, g).permute(1, 0, 2).reshape(b - a, hq)
            z = z.reshape(hkv, b - a, g).permute(1, 0, 2).reshape(b - a, hq)
            # running log-sum-exp merge of this level's partial into the accumulator
            m_old = m_acc[a:b]
            m_new = torch.maximum(m_old, m)
            c_old = torch.where(torch.isfinite(m_old), torch.exp(m_old - m_new), torch.zeros_like(m_old))
            c_new = torch.exp(m - m_new)
            o_acc[a:b] = o_acc[a:b] * c_old[..., None] + og * c_new[..., None]
            z_acc[a:b] = z_acc[a:b] * c_old + z * c_new
            m_acc[a:b] = m_new
    ok = z_acc > 0
    o = torch.where(ok[..., None], o_acc / torch.where(ok, z_acc, torch.ones_like(z_acc))[..., None],
                    torch.zeros_like(o_acc))
    lse = torch.where(ok, m_acc + torch.log(torch.where(ok, z_acc, torch.ones_like(z_acc))),
                      torch.full_like(z_acc, NEG_INF))
    return o, lse

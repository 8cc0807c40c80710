"""Random-init Llama-shaped decoder for the end-to-end beam-search harness.

The model math around attention (embeddings, RMSNorm, RoPE, projections,
SwiGLU MLP, LM head) is plain torch (hipBLASLt GEMMs); it is not part of the
decode hot path.  The reference runs the same structure through its modified
HF Llama (src/beam_engine/models/modeling_llama.py:428-562, 668-831): per
layer q/k/v projection, RoPE, append of the new K/V to the paged cache
(write_blocks_vectorized, :506-514), decode attention over the pages
(:517-525), output projection, MLP.  Here the append is ``PageTable`` (HIP
kernel) and attention is whatever ``attn(layer, q, kv_layer)`` the caller
passes (the HIP cascade / flat wrappers).

Prefill (prompt processing) follows the reference's order
(models/modeling_llama.py:213-283): the prompt's K/V is scattered into its
pages with one append per layer, then causal paged prefill attention over
those pages (``BatchPrefillWithPagedKVCacheWrapper``, HIP tile kernel with a
per-row causal limit) planned once for all layers.
"""

from __future__ import annotations

import gc
import math
from dataclasses import dataclass
from typing import Callable, List, Optional

import torch
import torch.nn.functional as F


@dataclass
class LlamaConfig:
    num_hidden_layers: int = 32
    hidden_size: int = 4096
    num_attention_heads: int = 32
    num_key_value_heads: int = 8
    head_dim: int = 128
    intermediate_size: int = 14336
    vocab_size: int = 128256
    rms_norm_eps: float = 1e-5
    rope_theta: float = 500000.0
    max_position_embeddings: int = 8192
    init_std: float = 0.02

    @staticmethod
    def llama3_8b() -> "LlamaConfig":
        return LlamaConfig()

    @staticmethod
    def tiny(layers: int = 2, vocab: int = 1000) -> "LlamaConfig":
        return LlamaConfig(num_hidden_layers=layers, hidden_size=256, num_attention_heads=8, num_key_value_heads=2,
                           head_dim=32, intermediate_size=512, vocab_size=vocab, max_position_embeddings=4096)

    def num_params(self) -> int:
        h, kvd = self.hidden_size, self.num_key_value_heads * self.head_dim
        per_layer = h * (h + 2 * kvd) + h * h + 3 * h * self.intermediate_size + 2 * h
        return self.num_hidden_layers * per_layer + 2 * self.vocab_size * h + h


class LlamaDecoder:
    """Weights ~ N(0, init_std) in ``dtype``; norms at 1."""

    def __init__(self, cfg: LlamaConfig, device="cuda", dtype=torch.bfloat16, seed: int = 0):
        self.cfg = cfg
        self.device = torch.device(device)
        self.dtype = dtype
        gen = torch.Generator(device=self.device).manual_seed(seed)
        h, hq, hkv, d = cfg.hidden_size, cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim

        def w(*shape):
            t = torch.empty(shape, device=self.device, dtype=dtype)
            t.normal_(0.0, cfg.init_std, generator=gen)
            return t

        self.embed = w(cfg.vocab_size, h)
        self.layers = []
        for _ in range(cfg.num_hidden_layers):
            self.layers.append(dict(
                ln1=torch.ones(h, device=self.device, dtype=dtype),
                wqkv=w((hq + 2 * hkv) * d, h),
                wo=w(h, hq * d),
                ln2=torch.ones(h, device=self.device, dtype=dtype),
                wgu=w(2 * cfg.intermediate_size, h),
                wd=w(h, cfg.intermediate_size),
            ))
        self.norm = torch.ones(h, device=self.device, dtype=dtype)
        self.lm_head = w(cfg.vocab_size, h)
        inv = 1.0 / (cfg.rope_theta ** (torch.arange(0, d, 2, dtype=torch.float64, device=self.device) / d))
        t = torch.arange(cfg.max_position_embeddings, dtype=torch.float64, device=self.device)
        freqs = torch.outer(t, inv)
        emb = torch.cat([freqs, freqs], dim=-1)
        self.cos = emb.cos().to(dtype)
        self.sin = emb.sin().to(dtype)

    # ---------------------------------------------------------------- pieces
    def _rms(self, x: torch.Tensor, wgt: torch.Tensor) -> torch.Tensor:
        return F.rms_norm(x, (x.shape[-1],), wgt, self.cfg.rms_norm_eps)

    @staticmethod
    def _rotate_half(x):
        x1, x2 = x.chunk(2, dim=-1)
        return torch.cat((-x2, x1), dim=-1)

    def _rope(self, x: torch.Tensor, pos: torch.Tensor) -> torch.Tensor:
        """x [..., T, H, D], pos [..., T] -> HF-style rotary embedding."""
        cos = self.cos[pos].unsqueeze(-2)
        sin = self.sin[pos].unsqueeze(-2)
        return x * cos + self._rotate_half(x) * sin

    def _qkv(self, layer, h):
        cfg = self.cfg
        hq, hkv, d = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        qkv = F.linear(h, layer["wqkv"])
        q = qkv[..., : hq * d].unflatten(-1, (hq, d))
        k = qkv[..., hq * d: (hq + hkv) * d].unflatten(-1, (hkv, d))
        v = qkv[..., (hq + hkv) * d:].unflatten(-1, (hkv, d))
        return q, k, v

    def _mlp(self, layer, x):
        h = self._rms(x, layer["ln2"])
        gu = F.linear(h, layer["wgu"])
        g, u = gu.chunk(2, dim=-1)
        return x + F.linear(F.silu(g) * u, layer["wd"])

    # ---------------------------------------------------------------- prefill
    @torch.no_grad()
    def prefill(self, input_ids: torch.Tensor, page_table, page_ids: List[List[int]]) -> torch.Tensor:
        """Prompts ``input_ids [R, S]`` (equal lengths); writes every prompt
        token's K/V into the request's pages; returns last-position logits [R, V]."""
        cfg = self.cfg
        r, s = input_ids.shape
        hq, hkv, d = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        ps = page_table.page_size
        pos = torch.arange(s, device=self.device).unsqueeze(0).expand(r, s)
        pages = torch.tensor([[p[i // ps] for i in range(s)] for p in page_ids], dtype=torch.int32,
                             device=self.device).reshape(-1)
        slots = (torch.arange(s, device=self.device, dtype=torch.int32) % ps).repeat(r)
        # causal paged prefill attention over the pages just written, planned
        # once for every layer (models/modeling_llama.py:775-798)
        from .attention import BatchPrefillWithPagedKVCacheWrapper
        npg = -(-s // ps)
        ws = torch.empty(256 << 20, dtype=torch.uint8, device=self.device)
        pre = BatchPrefillWithPagedKVCacheWrapper(ws)
        pre.plan([i * s for i in range(r + 1)], [i * npg for i in range(r + 1)],
                 [p[j] for p in page_ids for j in range(npg)], [s - (npg - 1) * ps] * r, hq, hkv, d, ps,
                 causal=True, q_data_type=self.dtype)
        x = F.embedding(input_ids, self.embed)
        for li, layer in enumerate(self.layers):
            h = self._rms(x, layer["ln1"])
            q, k, v = self._qkv(layer, h)
            q = self._rope(q, pos)
            k = self._rope(k, pos)
            page_table.write_blocks_vectorized(li, pages, k.reshape(r * s, hkv, d).contiguous(),
                                               v.reshape(r * s, hkv, d).contiguous(), slots)
            o = pre.run(q.reshape(r * s, hq, d), page_table.kv_cache_at_layer[li]).reshape(r, s, hq * d)
            x = x + F.linear(o, layer["wo"])
            x = self._mlp(layer, x)
        last = self._rms(x[:, -1], self.norm)
        return F.linear(last, self.lm_head)

    # ---------------------------------------------------------------- decode
    @torch.no_grad()
    def decode(self, token_ids: torch.Tensor, positions: torch.Tensor, write_pages: torch.Tensor,
               write_pos: torch.Tensor, page_table, attn: Callable, fused_rope: bool = True) -> torch.Tensor:
        """One token per candidate: ``token_ids/positions/write_pages/write_pos [N]``
        (device; positions int64, pages/slots int32).  ``attn(layer, q [N, Hq, D],
        kv_layer) -> o [N, Hq, D]``.  With ``fused_rope`` RoPE and the K/V append
        are one HIP kernel (bit-identical to the eager tensor code).  Returns
        logits [N, V]."""
        n = token_ids.shape[0]
        cfg = self.cfg
        x = F.embedding(token_ids, self.embed)
        for li, layer in enumerate(self.layers):
            h = self._rms(x, layer["ln1"])
            if fused_rope:
                qkv = F.linear(h, layer["wqkv"])
                q = page_table.write_rope_qkv(li, qkv, cfg.num_attention_heads, positions, self.cos, self.sin,
                                              write_pages, write_pos)
            else:
                q, k, v = self._qkv(layer, h)
                q = self._rope(q, positions)
                k = self._rope(k, positions)
                page_table.write_blocks_vectorized(li, write_pages, k, v, write_pos)
            o = attn(li, q, page_table.kv_cache_at_layer[li])
            x = x + F.linear(o.reshape(n, -1), layer["wo"])
            x = self._mlp(layer, x)
        return F.linear(self._rms(x, self.norm), self.lm_head)


def _align(nbytes: int, to: int = 256) -> int:
    return (nbytes + to - 1) // to * to


class GraphedDecoder:
    """Decode forward with the non-attention work captured as HIP graphs.

    Segment 0 = embedding + layer 0 up to its attention input (RMSNorm, fused
    q|k|v projection, fused RoPE + KV append); segment l = the rest of layer
    l-1 (output projection, residual, MLP) and layer l up to its attention
    input; the last segment ends with the final norm and the LM head.  The
    attention of every layer runs eagerly between two replays, from the plan
    of the current step, into a fixed output buffer.  Inputs (token ids,
    positions, write pages / slots) are copied into fixed device buffers
    before the replays; the graphs share one memory pool and are replayed in
    capture order.  ``capture_step`` also records the whole step, every
    layer's attention included, as one graph for plans of a fixed layout.
    """

    @staticmethod
    def header_bytes(n: int) -> int:
        """Bytes of a step-upload header for n candidates: the inputs (two
        int64 and two int32 rows) and a staged fork-copy list of 2n entries."""
        return _align(16 * n) + _align(8 * n) + _align(4 * (1 + 6 * n))

    def __init__(self, model: LlamaDecoder, page_table, n: int, header=None):
        cfg = model.cfg
        self.model, self.pt, self.n = model, page_table, n
        dev = model.device
        # inputs: token ids and positions (int64), write pages and slots (int32),
        # each pair one device buffer filled from pinned staging by one copy.
        # ``header``: (device, pinned host) uint8 views of header_bytes(n) at
        # the head of a step-upload block; the inputs and the staged copy list
        # then live there, and the block's owner uploads them with the plan
        self.header = header
        pin = dev.type == "cuda"
        if header is not None:
            hd, hh = header
            o32 = _align(16 * n)
            self._in64 = hd[: 16 * n].view(torch.long).view(2, n)
            self._in32 = hd[o32: o32 + 8 * n].view(torch.int32).view(2, n)
            self._h64 = hh[: 16 * n].view(torch.long).view(2, n)
            self._h32 = hh[o32: o32 + 8 * n].view(torch.int32).view(2, n)
            ocp = o32 + _align(8 * n)
            self.copy_list = (hd[ocp: ocp + 4 * (1 + 6 * n)].view(torch.int32),
                              hh[ocp: ocp + 4 * (1 + 6 * n)].view(torch.int32))
            # the header is carved from uninitialised memory: valid inputs (token
            # 0, position 0) until the first step stages its own
            self._in64.zero_()
            self._in32.zero_()
            self._h64.zero_()
            self._h32.zero_()
        else:
            self._in64 = torch.zeros((2, n), dtype=torch.long, device=dev)
            self._in32 = torch.zeros((2, n), dtype=torch.int32, device=dev)
            self._h64 = torch.zeros((2, n), dtype=torch.long, pin_memory=pin)
            self._h32 = torch.zeros((2, n), dtype=torch.int32, pin_memory=pin)
            self.copy_list = None
        self.tok, self.pos = self._in64[0], self._in64[1]
        self.wpg, self.wps = self._in32[0], self._in32[1]
        self._np = (self._h64.numpy(), self._h32.numpy())     # numpy views of the pinned staging
        self.o = torch.zeros((n, cfg.num_attention_heads, cfg.head_dim), dtype=model.dtype, device=dev)
        self.graphs = []
        self.q = []
        self.logits = None
        self._pool = None
        self.step_graph = None          # the whole step with its attention (capture_step)
        self.step_q: List[torch.Tensor] = []
        self.step_logits = None
        # page writes of the capture run go to a reserved page no candidate owns
        self._scratch_page = page_table.reserve_block(page_table.max_num_pages - 1)

    def _segment(self, l: int, x: Optional[torch.Tensor]):
        m, cfg = self.model, self.model.cfg
        if l == 0:
            x = F.embedding(self.tok, m.embed)
        else:
            prev = m.layers[l - 1]
            x = x + F.linear(self.o.reshape(self.n, -1), prev["wo"])
            x = m._mlp(prev, x)
        if l == cfg.num_hidden_layers:
            return x, None, F.linear(m._rms(x, m.norm), m.lm_head)
        layer = m.layers[l]
        h = m._rms(x, layer["ln1"])
        qkv = F.linear(h, layer["wqkv"])
        q = self.pt.write_rope_qkv(l, qkv, cfg.num_attention_heads, self.pos, m.cos, m.sin, self.wpg, self.wps)
        return x, q, None

    @torch.no_grad()
    def capture(self) -> None:
        L = self.model.cfg.num_hidden_layers
        # the warm-up pass below reads the inputs: token 0 at position 0, its
        # writes landing in a scratch slot; real steps overwrite the inputs
        self.tok.zero_()
        self.pos.zero_()
        self.wpg.fill_(self._scratch_page)
        self.wps.zero_()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):              # warm the libraries (hipBLASLt handles, workspaces)
            x = None
            for l in range(L + 1):
                x, _, _ = self._segment(l, x)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        self._pool = torch.cuda.graph_pool_handle()
        # No automatic garbage collection inside a capture: a collected pinned
        # host block or event is released with HIP calls that a capturing
        # stream forbids, and that error inside a destructor aborts the
        # process.  torch.cuda.graph still collects before each capture begins.
        gc_on = gc.isenabled()
        gc.collect()
        gc.disable()
        try:
            x = None
            for l in range(L + 1):
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g, pool=self._pool):
                    x, q, logits = self._segment(l, x)
                self.graphs.append(g)
                self.q.append(q)
                if logits is not None:
                    self.logits = logits
        finally:
            if gc_on:
                gc.enable()
        torch.cuda.synchronize()

    @torch.no_grad()
    def capture_step(self, attn_run: Callable) -> None:
        """One graph of the whole step: the page table's staged fork copies
        (when enabled: one counted launch over the list the last selection
        staged), every segment and, between them, each layer's attention
        launched by ``attn_run(layer, q, kv_layer, out)`` -- the launch of a
        fixed-layout plan (same device plan address and launch sizes for every
        step; the plan's contents are rewritten before each replay).  Needs
        ``capture`` first (its warm-up and memory pool)."""
        L = self.model.cfg.num_hidden_layers
        self.step_graph, self.step_q, self.step_logits = None, [], None
        gc_on = gc.isenabled()
        gc.collect()
        gc.disable()
        try:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, pool=self._pool):
                if self.pt.stage_copies_enabled:
                    self.pt.record_staged_copies()
                x = None
                for l in range(L + 1):
                    x, q, logits = self._segment(l, x)
                    if q is not None:
                        attn_run(l, q, self.pt.kv_cache_at_layer[l], self.o)
                        self.step_q.append(q)
            self.step_graph = g
            self.step_logits = logits
        finally:
            if gc_on:
                gc.enable()
        torch.cuda.synchronize()

    def run_step(self) -> torch.Tensor:
        """Replay the whole-step graph (inputs and the attention plan loaded);
        it performs the staged fork copies."""
        self.step_graph.replay()
        self.pt.consume_staged_copies()
        return self.step_logits

    def stage_inputs(self, tok, pos, wpg, wps, upload: bool = True) -> None:
        """Host arrays of the step's inputs -> the graphs' input buffers (two
        copies from pinned staging; the staging is rewritten only after the
        step's selection has synchronised).  ``upload=False``: only the pinned
        staging is written; the header's owner uploads it."""
        a, b = self._np
        a[0] = tok
        a[1] = pos
        b[0] = wpg
        b[1] = wps
        if upload:
            self._in64.copy_(self._h64, non_blocking=True)
            self._in32.copy_(self._h32, non_blocking=True)

    def load_inputs(self, tok, pos, wpg, wps) -> None:
        self.tok.copy_(tok, non_blocking=True)
        self.pos.copy_(pos, non_blocking=True)
        self.wpg.copy_(wpg, non_blocking=True)
        self.wps.copy_(wps, non_blocking=True)

    def run(self, attn: Callable) -> torch.Tensor:
        """``attn(layer, q, kv_layer, out)`` must write the layer's attention into ``out``."""
        L = self.model.cfg.num_hidden_layers
        self.graphs[0].replay()
        for l in range(L):
            attn(l, self.q[l], self.pt.kv_cache_at_layer[l], self.o)
            self.graphs[l + 1].replay()
        return self.logits

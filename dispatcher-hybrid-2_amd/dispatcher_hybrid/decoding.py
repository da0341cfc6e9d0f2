"""Incremental decoders: per-token cost O(log t) in the tree layers, flat in context.

Same classes, constructor arguments and public behaviour as the reference
(reference dispatcher_hybrid/decoding.py:50-488):

    IncrementalDecoder          exact, eager torch ops
    GraphedHybridDecoder        the whole step captured once as a HIP graph and replayed per token
    FusedGraphedHybridDecoder   graphed, with each tree layer's gate readouts + level recurrence as
                                ONE gfx950 kernel (dispatcher_hybrid.fused_step.decode_mixer_step)

All rows of a batch advance in lockstep (one shared position t). Tree-layer state per layer:
    B_hist  (B, Tmax, gh)     W1s.h1 of every position (the level-l source row is t - 2^l)
    rg_hist (B, Tmax, L, H)   transmit gates, stored at their source position
    V_ring  (B, S, d)         ring j (offset 2^(j+1)-2, 2^(j+1) slots) holds the state entering
                              level j for the last 2^(j+1) positions; S = 2^(L+1) - 2
Attention layers keep a (B, H, Tmax, hd) K/V cache with RoPE applied at the absolute position.
"""

import math
import warnings

import torch
import torch.nn.functional as F

from .modeling_dispatcher import (AttentionBlock, active_levels, causal_window_attention,
                                  level_gate_matmul, rope_rotate)


class _TreeLayerCache:
    """Decode state of one tree layer (layout: reference decoding.py:50-76)."""

    def __init__(self, mixer, batch, max_len, device, dtype):
        gh = mixer.gate_hidden.out_features
        self.L = L = mixer.levels
        self.H = H = mixer.num_heads
        self.hd = mixer.head_dim
        self.B_hist = torch.zeros(batch, max_len, gh, device=device, dtype=dtype)
        self.rg_hist = torch.zeros(batch, max_len, L, H, device=device, dtype=dtype)
        self.S = (2 << L) - 2
        self.V_ring = torch.zeros(batch, self.S, H * self.hd, device=device, dtype=dtype)
        self.offsets = torch.tensor([(2 << j) - 2 for j in range(L)], device=device)
        self.masks = torch.tensor([(2 << j) - 1 for j in range(L)], device=device)

    def slot(self, j, p):
        """Ring slot of position p (int or tensor) at level j."""
        return ((2 << j) - 2) + (p & ((2 << j) - 1))

    def write_slab(self, j, slab):
        """Store the level-j states of a (B, T, d) prefill slab. Only the last 2^(j+1) positions
        can still be read, and consecutive positions occupy distinct slots."""
        T = slab.shape[1]
        p0 = max(0, T - (2 << j))
        pos = torch.arange(p0, T, device=slab.device)
        self.V_ring[:, self.slot(j, pos)] = slab[:, p0:]


class _AttnCache:
    def __init__(self, attn, batch, max_len, device, dtype):
        self.k = torch.zeros(batch, attn.num_heads, max_len, attn.head_dim, device=device, dtype=dtype)
        self.v = torch.zeros_like(self.k)
        # materialised RoPE tables: graph capture needs stable device tensors to index
        self.rope_cos, self.rope_sin = attn.rope_tables(max_len, device, dtype)


def _check_single_document(model, idx):
    """The decoders apply the wrap mask only, not the doc-reset mask, so a prompt that spans
    documents would diverge from the parallel forward (reference decoding.py:89-98)."""
    if getattr(model.config, "doc_reset", False):
        if bool((idx == model.config.eot_token).any()):
            raise ValueError(
                f"prompt contains the document separator (token {model.config.eot_token}) and this "
                f"model was trained with doc_reset=True; the incremental decoders assume a single "
                f"document. Remove the separator, or use model.generate().")


class IncrementalDecoder:
    """Exact per-token decoder on eager torch ops.

        dec = IncrementalDecoder(model)
        logits = dec.prefill(ids)     # ids (T,) or (B, T) -> (T, V) or (B, T, V)
        logits = dec.step(tokens)     # (B,) or scalar -> (B, V) or (V,)
    """

    def __init__(self, model, max_len=None, dtype=None):
        self.m = model
        self.max_len = max_len or model.config.max_len
        param_dtype = next(model.parameters()).dtype
        # caches and activations share the weights' dtype; cast the model to pick precision
        if dtype is not None and dtype != param_dtype:
            raise ValueError(f"decoder dtype {dtype} != model dtype {param_dtype}; cast the "
                             f"model first, e.g. model.to(torch.bfloat16)")
        self.dtype = param_dtype
        self.device = next(model.parameters()).device
        self.caches = None
        self.batch = None
        self.t = 0

    def _alloc(self, batch):
        if self.caches is not None and self.batch == batch:
            return
        self.batch = batch
        self.caches = [
            _AttnCache(blk.attn, batch, self.max_len, self.device, self.dtype)
            if isinstance(blk, AttentionBlock) else
            _TreeLayerCache(blk.mixer, batch, self.max_len, self.device, self.dtype)
            for blk in self.m.blocks]

    # ---------- tree layer ----------
    def _tree_prefill(self, blk, cache, x):
        """Parallel mixer over the prompt that also fills B_hist, rg_hist and the rings
        (reference decoding.py:143-185)."""
        mx = blk.mixer
        Bb, T = x.shape[0], x.shape[1]
        L, H, hd = cache.L, cache.H, cache.hd
        h1 = blk.norm1(x)
        A = mx.gate_hidden(h1)
        Bs = mx.gate_hidden_src(h1)
        cache.B_hist[:, :T] = Bs
        n_lv = active_levels(L, T)
        V = mx.linear_in(h1).view(Bb, T, H, hd)
        cache.write_slab(0, V.reshape(Bb, T, H * hd))
        t = torch.arange(T, device=x.device)
        wrap = torch.stack([(t >= (1 << l)) for l in range(n_lv)], dim=1).to(x.dtype).unsqueeze(-1)
        lagged = torch.stack([torch.roll(Bs, shifts=1 << l, dims=1) for l in range(n_lv)], dim=2)
        hidden = torch.relu(A.unsqueeze(2) + lagged * wrap) ** 2
        pre_i, pre_f, pre_r = (level_gate_matmul(hidden, W[:n_lv]) + b[:n_lv]
                               for W, b in mx._gate_params())
        ig = torch.sigmoid(pre_i) * wrap
        fg = torch.sigmoid(pre_f) * wrap + (1.0 - wrap)
        rg = torch.sigmoid(pre_r)
        cache.rg_hist[:, :T, :n_lv] = rg
        if n_lv < L:
            # levels beyond the prompt's horizon send no message yet, but later tokens read the
            # transmit gates of these positions at those levels
            hid0 = torch.relu(A) ** 2
            for l in range(n_lv, L):
                cache.rg_hist[:, :T, l] = torch.sigmoid(F.linear(hid0, mx.reset_out[l]) + mx.reset_out_bias[l])
        for l in range(n_lv):
            msg = torch.roll(rg[:, :, l].unsqueeze(-1) * V, shifts=1 << l, dims=1)
            V = fg[:, :, l].unsqueeze(-1) * V + ig[:, :, l].unsqueeze(-1) * msg
            if l + 1 < L:
                cache.write_slab(l + 1, V.reshape(Bb, T, H * hd))
        for j in range(n_lv + 1, L):                  # beyond the horizon the state passes through
            cache.write_slab(j, V.reshape(Bb, T, H * hd))
        x = x + mx.linear_out(V.reshape(Bb, T, H * hd))
        return x + blk.ffn(blk.norm2(x))

    def _tree_step(self, blk, cache, x, t):
        """One position through a tree layer (reference decoding.py:187-222)."""
        mx = blk.mixer
        Bb = x.shape[0]
        L, H, hd = cache.L, cache.H, cache.hd
        h1 = blk.norm1(x)
        A = mx.gate_hidden(h1)
        cache.B_hist[:, t] = mx.gate_hidden_src(h1)
        V = mx.linear_in(h1).view(Bb, H, hd)
        cache.V_ring[:, cache.slot(0, t)] = V.reshape(Bb, -1)
        lev = torch.arange(L, device=x.device)
        src = t - torch.pow(2, lev)
        ok = src >= 0
        src_c = src.clamp(min=0)
        okf = ok.view(1, L, 1)
        hid = torch.relu(A.unsqueeze(1) + cache.B_hist[:, src_c] * okf) ** 2        # (B, L, gh)
        gates = [level_gate_matmul(hid.unsqueeze(1), W)[:, 0] + b for W, b in mx._gate_params()]
        i_ = torch.sigmoid(gates[0]) * okf
        f_ = torch.sigmoid(gates[1])
        f_ = f_ * okf + (~okf).to(f_.dtype)                                         # masked: f = 1
        r_ = torch.sigmoid(gates[2])
        cache.rg_hist[:, t] = r_
        rg_src = cache.rg_hist[:, src_c, lev]                                       # (B, L, H)
        V_src = cache.V_ring[:, cache.offsets + (src_c & cache.masks)].view(Bb, L, H, hd)
        msg = rg_src.unsqueeze(-1) * V_src
        for l in range(L):
            V = f_[:, l].unsqueeze(-1) * V + i_[:, l].unsqueeze(-1) * msg[:, l]
            if l + 1 < L:
                cache.V_ring[:, cache.slot(l + 1, t)] = V.reshape(Bb, -1)
        x = x + mx.linear_out(V.reshape(Bb, -1))
        return x + blk.ffn(blk.norm2(x))

    # ---------- attention layer ----------
    def _attn_prefill(self, blk, cache, x):
        at = blk.attn
        Bb, T = x.shape[0], x.shape[1]
        h1 = blk.norm1(x)
        shape = (Bb, T, at.num_heads, at.head_dim)
        q = at.apply_rope(at.linear_q(h1).view(shape).transpose(1, 2), T)
        k = at.apply_rope(at.linear_k(h1).view(shape).transpose(1, 2), T)
        v = at.linear_v(h1).view(shape).transpose(1, 2)
        cache.k[:, :, :T] = k
        cache.v[:, :, :T] = v
        window = at.window if 0 < at.window < T else 0
        y = causal_window_attention(q, k, v, window)
        x = x + at.linear_out(y.transpose(1, 2).reshape(Bb, T, at.embed_dim))
        return x + blk.ffn(blk.norm2(x))

    def _attn_step(self, blk, cache, x, t):
        at = blk.attn
        Bb = x.shape[0]
        h1 = blk.norm1(x)
        cos, sin = cache.rope_cos[t], cache.rope_sin[t]
        q = rope_rotate(at.linear_q(h1).view(Bb, at.num_heads, at.head_dim), cos, sin)
        cache.k[:, :, t] = rope_rotate(at.linear_k(h1).view(Bb, at.num_heads, at.head_dim), cos, sin)
        cache.v[:, :, t] = at.linear_v(h1).view(Bb, at.num_heads, at.head_dim)
        lo = max(0, t + 1 - at.window) if at.window > 0 else 0
        k = cache.k[:, :, lo:t + 1]
        v = cache.v[:, :, lo:t + 1]
        scores = torch.matmul(k, q.unsqueeze(-1)).squeeze(-1) / math.sqrt(at.head_dim)
        att = torch.softmax(scores, dim=-1)                      # model-dtype softmax, as eager
        y = torch.matmul(att.unsqueeze(2), v).squeeze(2).reshape(Bb, -1)
        x = x + at.linear_out(y)
        return x + blk.ffn(blk.norm2(x))

    # ---------- public ----------
    @torch.no_grad()
    def prefill(self, idx):
        """idx: (T,) or (B, T) token ids. Returns (T, vocab) or (B, T, vocab) logits."""
        self._squeeze = idx.dim() == 1
        ids = idx.view(1, -1) if self._squeeze else idx
        _check_single_document(self.m, ids)
        if ids.shape[1] > self.max_len:
            raise ValueError(f"prompt of {ids.shape[1]} exceeds max_len {self.max_len}")
        self._alloc(ids.shape[0])
        x = self.m.embedding(ids).to(self.dtype)
        for blk, cache in zip(self.m.blocks, self.caches):
            x = (self._attn_prefill(blk, cache, x) if isinstance(blk, AttentionBlock)
                 else self._tree_prefill(blk, cache, x))
        self.t = ids.shape[1]
        out = self.m.lm_head(self.m.norm_out(x))
        return out[0] if self._squeeze else out

    @torch.no_grad()
    def step(self, tokens):
        """tokens: scalar, (1,) or (B,). Returns (vocab,) or (B, vocab) logits."""
        if self.t >= self.max_len:
            raise ValueError(f"context exhausted at max_len {self.max_len}")
        t = self.t
        toks = tokens.view(-1)
        if toks.shape[0] != self.batch and not (self.batch == 1 and toks.shape[0] == 1):
            raise ValueError(f"got {toks.shape[0]} tokens for batch {self.batch}")
        x = self.m.embedding(toks).to(self.dtype)
        for blk, cache in zip(self.m.blocks, self.caches):
            x = (self._attn_step(blk, cache, x, t) if isinstance(blk, AttentionBlock)
                 else self._tree_step(blk, cache, x, t))
        self.t = t + 1
        out = self.m.lm_head(self.m.norm_out(x))
        return out[0] if self._squeeze else out


# ==============================================================================================
# Graph-replayed decoders. The per-token work is small and launch-bound, so the whole step is
# captured once (after an eager prefill) and replayed per token. The position lives on the device
# (t_buf) so one graph serves every position; attention reads the full padded cache under a
# validity mask so its shapes are capture-stable.
# ==============================================================================================


class _FusedPrefillDecoder(IncrementalDecoder):
    """The fused decoder's prefill: each tree layer runs the parallel gfx950 kernels -- activated
    gates of all L levels in one launch, the level scan over the active levels in a second, which
    also stores the ring slabs -- instead of the eager roll/level loop, and fills the same state
    (B_hist, rg_hist for every level, V_ring; reference decoding.py:143-185). Attention layers (bf16,
    head width 32/64/128) run the banded-attention kernel, which also writes rope(k) and v into the
    caches; the steps stay those of IncrementalDecoder."""

    def _attn_prefill(self, blk, cache, x):
        from . import fused_attention as fa
        at = blk.attn
        if not (fa.supported(x.dtype, at.head_dim) and cache.k.dtype == x.dtype):
            return super()._attn_prefill(blk, cache, x)
        T = x.shape[1]
        h1 = blk.norm1(x)
        window = at.window if 0 < at.window < T else 0
        cos, sin = at.rope_tables(T, x.device, x.dtype)
        y = fa.window_attention(at.linear_q(h1), at.linear_k(h1), at.linear_v(h1), cos, sin, at.num_heads,
                                window, k_cache=cache.k, v_cache=cache.v)
        x = x + at.linear_out(y)
        return x + blk.ffn(blk.norm2(x))

    def _tree_prefill(self, blk, cache, x):
        from .fused_gates import input_projections, prefill_gate_scan
        mx = blk.mixer
        T = x.shape[1]
        dt = cache.V_ring.dtype
        h1 = blk.norm1(x)
        V0, A, Bs = input_projections(h1, mx)
        cache.B_hist[:, :T] = Bs
        (Wi, bi), (Wf, bf), (Wr, br) = mx._gate_params()
        V = prefill_gate_scan(A.to(dt), Bs.to(dt), Wi, Wf, Wr, bi, bf, br, V0.to(dt), cache.H,
                              cache.rg_hist, cache.V_ring)
        x = x + mx.linear_out(V.to(x.dtype))
        return x + blk.ffn(blk.norm2(x))


class _GraphedBase:
    def _capture(self, step_fn, attr="graph"):
        g = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        tok = self.token_buf.clone()
        with torch.cuda.stream(side):
            for _ in range(3):                      # warm-ups: allocator pools, library handles
                step_fn()
                self.t_buf.fill_(self.t)            # undo the warm-up's position advance
                self.token_buf.copy_(tok)           # and a fused greedy pick's token
        torch.cuda.current_stream().wait_stream(side)
        with torch.cuda.graph(g):
            step_fn()
        setattr(self, attr, g)

    @torch.no_grad()
    def step(self, tokens):
        if self.t >= self.max_len:
            raise ValueError(f"context exhausted at max_len {self.max_len}")
        self.token_buf.copy_(tokens.view(-1))
        self.graph.replay()
        self.t += 1
        # the graph overwrites logits_out on the next replay: hand out a copy
        out = self.logits_out.clone()
        return out[0] if self._squeeze else out


class GraphedHybridDecoder(_GraphedBase):
    """Eager prefill, then one HIP-graph replay per generated token."""

    _prefill_cls = IncrementalDecoder

    def __init__(self, model, max_len=None, dtype=None):
        if not torch.cuda.is_available():
            raise RuntimeError("GraphedHybridDecoder requires a GPU")
        self.inner = self._prefill_cls(model, max_len, dtype=dtype)
        self.m = model
        self.max_len = self.inner.max_len
        self.dtype = self.inner.dtype
        self.t = 0

    @torch.no_grad()
    def prefill(self, idx):
        out = self.inner.prefill(idx)
        self._squeeze = self.inner._squeeze
        self.t = self.inner.t
        dev = next(self.m.parameters()).device
        Bb = self.inner.batch
        self.token_buf = torch.zeros(Bb, dtype=torch.long, device=dev)
        self.t_buf = torch.full((1,), self.t, dtype=torch.long, device=dev)
        self.logits_out = torch.zeros(Bb, self.m.lm_head.out_features, device=dev, dtype=self.dtype)
        self.arangeT = torch.arange(self.max_len, device=dev)
        self._prepare()
        self._capture(self._step_all)
        return out

    def _prepare(self):
        # level-major transposed gate weights (L, gh, H) for the batched readout bmm
        self._gate_wt = {}
        for i, blk in enumerate(self.m.blocks):
            if hasattr(blk, "mixer"):
                self._gate_wt[i] = [W.transpose(1, 2).contiguous() for W, _ in blk.mixer._gate_params()]

    def _tree_step_g(self, i, blk, cache, x):
        mx = blk.mixer
        Bb = x.shape[0]
        L, H, hd = cache.L, cache.H, cache.hd
        dev = x.device
        h1 = blk.norm1(x)
        A = mx.gate_hidden(h1)
        cache.B_hist.index_copy_(1, self.t_buf, mx.gate_hidden_src(h1).unsqueeze(1))
        V = mx.linear_in(h1).view(Bb, H, hd)
        lev = torch.arange(L, device=dev)
        src = self.t_buf - torch.pow(2, lev)
        ok = src >= 0
        src_c = src.clamp(min=0)
        okf = ok.view(1, L, 1)
        hid = torch.relu(A.unsqueeze(1) + cache.B_hist.index_select(1, src_c) * okf) ** 2  # (B, L, gh)
        hid_l = hid.transpose(0, 1).contiguous()                                          # (L, B, gh)
        (_, bi), (_, bf), (_, br) = mx._gate_params()
        wi, wf, wr = self._gate_wt[i]
        i_ = torch.sigmoid(torch.bmm(hid_l, wi).transpose(0, 1) + bi) * okf
        f_ = torch.sigmoid(torch.bmm(hid_l, wf).transpose(0, 1) + bf)
        f_ = f_ * okf + (~okf).to(f_.dtype)
        r_ = torch.sigmoid(torch.bmm(hid_l, wr).transpose(0, 1) + br)
        cache.rg_hist.index_copy_(1, self.t_buf, r_.unsqueeze(1))
        rg_src = cache.rg_hist.index_select(1, src_c)[:, lev, lev]
        V_src = cache.V_ring.index_select(1, cache.offsets + (src_c & cache.masks)).view(Bb, L, H, hd)
        msg = rg_src.unsqueeze(-1) * V_src
        levs = [V.reshape(Bb, -1)]
        for l in range(L):                          # unrolled at capture time
            V = f_[:, l].unsqueeze(-1) * V + i_[:, l].unsqueeze(-1) * msg[:, l]
            if l + 1 < L:
                levs.append(V.reshape(Bb, -1))
        slots_w = cache.offsets + (self.t_buf & cache.masks)
        cache.V_ring.index_copy_(1, slots_w, torch.stack(levs, dim=1))
        x = x + mx.linear_out(V.reshape(Bb, -1))
        return x + blk.ffn(blk.norm2(x))

    def _attn_step_g(self, blk, cache, x):
        at = blk.attn
        Bb = x.shape[0]
        h1 = blk.norm1(x)
        cos = cache.rope_cos.index_select(0, self.t_buf)[0]
        sin = cache.rope_sin.index_select(0, self.t_buf)[0]
        q = rope_rotate(at.linear_q(h1).view(Bb, at.num_heads, at.head_dim), cos, sin)
        k_new = rope_rotate(at.linear_k(h1).view(Bb, at.num_heads, at.head_dim), cos, sin)
        cache.k.index_copy_(2, self.t_buf, k_new.unsqueeze(2))
        cache.v.index_copy_(2, self.t_buf, at.linear_v(h1).view(Bb, at.num_heads, at.head_dim).unsqueeze(2))
        valid = self.arangeT <= self.t_buf
        if at.window > 0:
            valid = valid & (self.arangeT > self.t_buf - at.window)
        scores = torch.matmul(cache.k, q.unsqueeze(-1)).squeeze(-1) / math.sqrt(at.head_dim)  # (B, H, Tmax)
        scores = scores.masked_fill(~valid.view(1, 1, -1), float("-inf"))
        att = torch.softmax(scores.float(), dim=-1).to(x.dtype)
        y = torch.matmul(att.unsqueeze(2), cache.v).squeeze(2).reshape(Bb, -1)
        x = x + at.linear_out(y)
        return x + blk.ffn(blk.norm2(x))

    def _step_all(self):
        x = self.m.embedding(self.token_buf).to(self.dtype)
        for i, (blk, cache) in enumerate(zip(self.m.blocks, self.inner.caches)):
            x = (self._attn_step_g(blk, cache, x) if isinstance(blk, AttentionBlock)
                 else self._tree_step_g(i, blk, cache, x))
        self.logits_out.copy_(self.m.lm_head(self.m.norm_out(x)))
        self.t_buf.add_(1)


class FusedGraphedHybridDecoder(GraphedHybridDecoder):
    """Graphed decoder on gfx950 kernels. Prefill: the parallel gate kernels fill the tree state
    (_FusedPrefillDecoder). Step: per tree layer six launches (five at batch 1, where the
    recurrence runs inside the out-projection launch, dh_decode_scan_out)

        dh_decode_gemv       RMSNorm1 + [W_in; W1x; W1s] -> V0, A, B_hist[t]
        dh_decode_gates      gate readouts of all L levels, one wave per (level, head)
        dh_decode_scan       the level recurrence over the rings
        dh_decode_gemv       linear_out + residual
        dh_decode_gemv       RMSNorm2 + [W_gate; W_up] + SwiGLU
        dh_decode_gemv       linear_down + residual

    in place of ~17 torch ops, the embedding gather folded into the first launch and RMSNorm_out +
    lm_head as one launch. An attention layer is the same chain with dh_decode_gemv for its
    projections and one dh_decode_attention launch (RoPE, cache write, windowed softmax, value
    average) in place of the mixer. Same caches, same graph harness; raises ImportError when the
    kernel library is missing.
    """

    _prefill_cls = _FusedPrefillDecoder

    def __init__(self, model, max_len=None, dtype=None, persistent=True):
        from . import fused_step                          # loads libdh_mixer.so
        self._fused_step = fused_step
        # batch-1 bf16 greedy steps as one cooperative launch each (dh_decode_persistent_step)
        # where the model fits it; False keeps the graph of launches
        self.use_persistent = persistent
        self._pers = None
        # one-launch steps between status checks (each check synchronises); 0: only check_persistent()
        self.persistent_check_every = 64
        self._pers_unchecked = 0
        super().__init__(model, max_len, dtype)

    def _prepare(self):
        super()._prepare()
        # the one-launch step's layer table holds raw addresses of this prefill's caches: a new
        # prefill (possibly another batch, reallocating them) derives it again
        self._pers = None
        dev = next(self.m.parameters()).device
        cfg = self.m.config
        Bb, dt = self.inner.batch, self.dtype
        mix0 = next(b.mixer for b in self.m.blocks if hasattr(b, "mixer"))
        gh = mix0.gate_hidden.out_features
        z = lambda n: torch.zeros(Bb, n, device=dev, dtype=dt)
        self.x_buf = z(cfg.d_model)            # residual stream
        self.v0_buf, self.y_buf = z(cfg.d_model), z(cfg.d_model)
        self.a_buf = z(gh)
        self.h_buf = z(cfg.dim_feedforward)
        self.q_buf, self.k_buf, self.v_buf = z(cfg.d_model), z(cfg.d_model), z(cfg.d_model)
        # staging of the two-launch mixer step, shared by every tree layer (same shapes)
        self.stage = torch.zeros(self._fused_step.stage_floats(Bb, mix0.num_heads, mix0.levels,
                                                               mix0.head_dim), device=dev)
        # small batches split each head's attention window over several workgroups
        # greedy decoding on the device: the step's vocabulary head also writes argmax candidates
        # (batch 1) and a second graph ends with the pick, which becomes the next step's input
        self._greedy_graph = None
        self._greedy_capture = False
        self.tok_hist = torch.zeros(Bb, self.max_len + 1, dtype=torch.long, device=dev)
        self.cand = None
        if Bb == 1:
            self.cand = self._fused_step.candidate_buffer(dt, self.logits_out.shape[1], cfg.d_model, 1, dev)
        att0 = next((b.attn for b in self.m.blocks if isinstance(b, AttentionBlock)), None)
        self.attn_ws = None
        if att0 is not None and Bb * att0.num_heads <= 64:
            self.attn_ws = self._fused_step.attention_workspace(Bb, att0.num_heads, att0.head_dim, dev)

    def _persistent_setup(self):
        """Layer table and scratch of the one-launch step (a dict), or False when this decoder cannot use it
        (batch > 1, fp32, or dimensions outside the kernel's)."""
        fs, m = self._fused_step, self.m
        cfg = m.config
        if self.inner.batch != 1 or self.dtype != torch.bfloat16:
            return False
        dev = next(m.parameters()).device
        eps = {self._eps(n, self.dtype) for n in [b.norm1 for b in m.blocks] + [b.norm2 for b in m.blocks]
               + [m.norm_out]}
        if len(eps) != 1:
            return False
        rows, kinds = [], []
        dims = None
        for blk, cache in zip(m.blocks, self.inner.caches):
            f = blk.ffn
            w = [0] * fs.LAYER_WORDS
            w[1] = blk.norm1.weight
            w[15], w[16], w[17], w[18] = blk.norm2.weight, f.linear_gate.weight, f.linear_up.weight, f.linear_down.weight
            if isinstance(blk, AttentionBlock):
                at = blk.attn
                span = min(at.window, self.max_len) if at.window > 0 else self.max_len
                if at.head_dim != 64 or span > fs.MAX_WINDOW:
                    return False
                kinds.append(1)
                w[0] = 1
                w[2], w[3], w[4], w[5] = at.linear_q.weight, at.linear_k.weight, at.linear_v.weight, at.linear_out.weight
                w[6], w[7], w[8], w[9] = cache.k, cache.v, cache.rope_cos, cache.rope_sin
                w[10] = int(at.window)
            else:
                mx = blk.mixer
                kinds.append(0)
                w[2], w[3], w[4] = mx.linear_in.weight, mx.gate_hidden.weight, mx.gate_hidden_src.weight
                w[5], w[6], w[7] = mx.gate_out, mx.forget_out, mx.reset_out
                w[8], w[9], w[10] = mx.gate_out_bias, mx.forget_out_bias, mx.reset_out_bias
                w[11], w[12], w[13], w[14] = mx.linear_out.weight, cache.B_hist, cache.rg_hist, cache.V_ring
                dims = (cfg.d_model, mx.gate_hidden.out_features, mx.num_heads, mx.head_dim, mx.levels)
            for i, v in enumerate(w):
                if isinstance(v, torch.Tensor):
                    if v.dtype != self.dtype or not v.is_contiguous():
                        return False
                    w[i] = v.data_ptr()
            rows.append(w)
        if dims is None:
            return False
        d, GH, H, hd, L = dims
        ff, V = cfg.dim_feedforward, self.logits_out.shape[1]
        grid = torch.cuda.get_device_properties(dev).multi_processor_count
        if not fs.persistent_fits(d, GH, H, hd, L, ff, grid):
            return False
        emb = m.lm_head.weight
        if emb.data_ptr() != m.embedding.weight.data_ptr() or not emb.is_contiguous() or emb.dtype != self.dtype:
            return False                                   # the kernel reads one tied table
        nbytes = fs.persistent_scratch_bytes(d, GH, H, L, ff, grid)
        scratch = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
        table = torch.tensor(rows, dtype=torch.int64, device=dev)
        return dict(table=table, kinds=kinds, emb=emb, norm_out=m.norm_out.weight, eps=eps.pop(),
                    dims=(d, GH, H, hd, L, ff, V, self.max_len), scratch=scratch)

    def _persistent_step(self):
        p = self._pers
        self._fused_step.persistent_step(p["table"], p["kinds"], p["emb"], p["norm_out"], p["eps"], p["dims"],
                                         self.t_buf, self.token_buf, self.tok_hist, self.logits_out, p["scratch"])

    def persistent_status(self):
        """(timed out, first failing phase + 1) of this decoder's one-launch steps (synchronises);
        (0, 0) when none ran or all completed."""
        if not self._pers:
            return 0, 0
        return self._fused_step.persistent_status(self._pers["scratch"])

    def check_persistent(self):
        """Verify the one-launch steps issued since the last check (synchronises). Returns the number
        of steps redone.

        A one-launch step assumes every workgroup of its launch is resident at once; should one not
        be (other work on the device), a bounded wait times out, the launch ends without advancing
        t_buf or writing a token, and every later launch on the same scratch stops at its first wait.
        Everything a step writes is a function of its token, its position and the state before it,
        so the steps from the device position on are redone through the graph of launches, which
        this decoder then keeps using. The status is cleared and the tag epoch advanced, so no word
        of the aborted launches can match a later tag."""
        self._pers_unchecked = 0
        flag, phase = self.persistent_status()
        if not flag:
            return 0
        scratch = self._pers["scratch"]
        t_dev = int(self.t_buf.item())
        scratch[8:16].zero_()                              # status words
        scratch[0:8].view(torch.int64).add_(1)             # tag epoch
        warnings.warn(f"dh_decode_persistent_step: a wait timed out in phase {phase % 1000 - 1} at position "
                      f"{t_dev}; redoing {self.t - t_dev} step(s) through the graph of launches, which this "
                      f"decoder uses from now on", RuntimeWarning)
        self.use_persistent = False
        self._pers = False
        redo, self.t = self.t - t_dev, t_dev
        for _ in range(redo):
            self.step_greedy()
        return redo

    @staticmethod
    def _eps(norm, dtype):
        # nn.RMSNorm(eps=None) takes the epsilon of torch's math type, fp32 for fp32 and bf16 inputs
        return norm.eps if norm.eps is not None else torch.finfo(torch.float32).eps

    def _ffn_g(self, blk):
        fs = self._fused_step
        f, d = blk.ffn, self.x_buf.shape[1]
        ff = self.h_buf.shape[1]
        fs.decode_gemv(self.x_buf, [(f.linear_gate.weight, self.h_buf, ff, 0),
                                    (f.linear_up.weight, self.h_buf, ff, 0)], self.t_buf,
                       norm_weight=blk.norm2.weight, eps=self._eps(blk.norm2, self.dtype), swiglu=True)
        fs.decode_gemv(self.h_buf, [(f.linear_down.weight, self.x_buf, d, 0)], self.t_buf,
                       resid=self.x_buf)

    def _input(self, first):
        """The block's input rows: the embedding rows of the tokens for the first block."""
        if first:
            return self.m.embedding.weight, self.token_buf
        return self.x_buf, None

    def _tree_step_f(self, blk, cache, first):
        fs = self._fused_step
        mx = blk.mixer
        d, gh = self.x_buf.shape[1], self.a_buf.shape[1]
        x_in, rows = self._input(first)
        fs.decode_gemv(x_in, [(mx.linear_in.weight, self.v0_buf, d, 0),
                              (mx.gate_hidden.weight, self.a_buf, gh, 0),
                              (mx.gate_hidden_src.weight, cache.B_hist, cache.B_hist.stride(0), gh)],
                       self.t_buf, norm_weight=blk.norm1.weight, eps=self._eps(blk.norm1, self.dtype),
                       x_rows=rows)
        gate_args = (self.a_buf, cache.B_hist, mx.gate_out, mx.forget_out, mx.reset_out, mx.gate_out_bias,
                     mx.forget_out_bias, mx.reset_out_bias, self.t_buf, cache.rg_hist, cache.V_ring,
                     self.v0_buf, self.y_buf, self.stage)
        if fs.scan_out_supported(self.x_buf.shape[0], d):
            # batch 1: the recurrence runs inside the out-projection launch
            fs.decode_gates_scan_out(*gate_args, mx.linear_out.weight, x_in, self.x_buf, resid_rows=rows)
        else:
            fs.decode_gates_scan(*gate_args)
            fs.decode_gemv(self.y_buf, [(mx.linear_out.weight, self.x_buf, d, 0)], self.t_buf,
                           resid=x_in, resid_rows=rows)
        self._ffn_g(blk)

    def _attn_step_f(self, blk, cache, first):
        fs = self._fused_step
        at = blk.attn
        Bb, d = self.x_buf.shape
        x_in, rows = self._input(first)
        fs.decode_gemv(x_in, [(at.linear_q.weight, self.q_buf, d, 0), (at.linear_k.weight, self.k_buf, d, 0),
                              (at.linear_v.weight, self.v_buf, d, 0)], self.t_buf,
                       norm_weight=blk.norm1.weight, eps=self._eps(blk.norm1, self.dtype), x_rows=rows)
        fs.decode_attention(self.q_buf, self.k_buf, self.v_buf, cache.rope_cos, cache.rope_sin,
                            cache.k, cache.v, self.t_buf, self.y_buf, at.window, workspace=self.attn_ws)
        fs.decode_gemv(self.y_buf, [(at.linear_out.weight, self.x_buf, d, 0)], self.t_buf,
                       resid=x_in, resid_rows=rows)
        self._ffn_g(blk)

    def _step_all(self):
        for i, (blk, cache) in enumerate(zip(self.m.blocks, self.inner.caches)):
            if isinstance(blk, AttentionBlock):
                self._attn_step_f(blk, cache, i == 0)
            else:
                self._tree_step_f(blk, cache, i == 0)
        V = self.logits_out.shape[1]
        fs = self._fused_step
        cand = self.cand if self._greedy_capture else None
        # the last launch also advances the device position (no separate add kernel)
        fs.decode_gemv(self.x_buf, [(self.m.lm_head.weight, self.logits_out, V, 0)], self.t_buf,
                       norm_weight=self.m.norm_out.weight, eps=self._eps(self.m.norm_out, self.dtype),
                       t_advance=self.t_buf, argmax_cand=cand)
        if self._greedy_capture:
            # greedy pick into the next step's token input and the token history (at the new position)
            if cand is not None:
                fs.argmax_reduce(cand, self.token_buf, self.t_buf, self.tok_hist)
            else:
                fs.argmax_tokens(self.logits_out, out=self.token_buf)
                self.tok_hist.index_copy_(1, self.t_buf, self.token_buf.unsqueeze(1))

    @torch.no_grad()
    def greedy_start(self, logits):
        """Start device-side greedy decoding after prefill: the argmax of `logits` (the prefill's
        last-position logits, (B, V) or (V,)) becomes the token fed to the next step and the first
        entry of tok_hist (at the current position)."""
        lg = logits.view(-1, logits.shape[-1])
        self._fused_step.argmax_tokens(lg, out=self.token_buf)
        self.tok_hist[:, self.t] = self.token_buf

    @torch.no_grad()
    def step_greedy(self):
        """One decode step fed by the token in token_buf, ending with the greedy pick: the next token
        goes to token_buf and to tok_hist[:, t + 1] on the device -- one graph replay, no host work
        per token (what fast_generate's greedy branch runs; same tokens as argmax of step())."""
        if self.t >= self.max_len:
            raise ValueError(f"context exhausted at max_len {self.max_len}")
        if self.use_persistent and self._pers is None:
            self._pers = self._persistent_setup()
        if self.use_persistent and self._pers:
            self._persistent_step()
            self.t += 1
            self._pers_unchecked += 1
            if self.persistent_check_every and self._pers_unchecked >= self.persistent_check_every:
                self.check_persistent()
            return
        if self._greedy_graph is None:
            self._greedy_capture = True
            try:
                self._capture(self._step_all, attr="_greedy_graph")
            finally:
                self._greedy_capture = False
        self._greedy_graph.replay()
        self.t += 1

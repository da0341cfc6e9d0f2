"""Incremental decoders: per-token cost O(log t) in the tree layers, flat in context.

The reference's classes, constructor arguments and public behaviour (reference
dispatcher_hybrid/decoding.py:50-488):

    IncrementalDecoder          one position per step on eager torch ops
    GraphedHybridDecoder        the same step captured once as a HIP graph, replayed per token
    FusedGraphedHybridDecoder   graphed, the step on gfx950 kernels (fused_step): per tree layer the
                                gate readouts, the level recurrence over the rings and the GEMV chain;
                                at batch 1 in bf16, greedy steps as one launch each

Design. A decoder keeps one state object per layer (_TreeLayerCache, _AttnCache), and builds both
halves of decoding from the model's own modules:
  * prefill runs the model's parallel forward over the prompt (the mixer's eager path with the wrap
    mask, or the fused kernels), and each layer hands the state a decoder keeps -- W1s rows,
    transmit gates, the state entering every level, rotated keys and values -- to its state object
    through a recorder;
  * a step is one position through every layer, every cache addressed through a DEVICE position
    tensor (index_select / index_copy_). The eager decoder writes the position before each step;
    the graphed decoder captures the very same step once and advances the position on the device,
    so eager and graphed run identical arithmetic and return identical logits.

All rows of a batch advance in lockstep (one shared position t). Tree-layer state (the reference's
tensors and slot arithmetic, so the state is interchangeable with its decoders):
    B_hist  (B, Tmax, gh)     W1s.h1 of every position (the level-l source row is t - 2^l)
    rg_hist (B, Tmax, L, H)   transmit gates, stored at their source position
    V_ring  (B, S, d)         ring j (offset 2^(j+1)-2, 2^(j+1) slots) holds the state entering
                              level j for the last 2^(j+1) positions; S = 2^(L+1) - 2
Attention layers keep rotated keys and values head-major, (B, H, Tmax, hd) in `keys` / `values`;
`k` / `v` are views of them in the reference's (B, Tmax, H, hd) indexing.
"""

import math
import warnings

import torch
import torch.nn.functional as F

from .modeling_dispatcher import AttentionBlock, active_levels, level_gate_matmul, rope_rotate


class _TreeLayerCache:
    """Decode state of one tree layer and the per-token step that advances it."""

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
        self.lags = torch.tensor([1 << j for j in range(L)], device=device)
        # position-major index of (source position, level) in rg_hist viewed as (B, Tmax * L, H)
        self.level_ids = torch.arange(L, device=device)
        self.readout_t = None

    def slot(self, j, p):
        """Ring slot of position p (int or tensor) at level j."""
        return ((2 << j) - 2) + (p & ((2 << j) - 1))

    def write_slab(self, j, slab):
        """Keep the level-j states of a (B, T, d) prompt slab: the last 2^(j+1) positions, which
        occupy distinct slots of ring j."""
        T = slab.shape[1]
        p0 = max(0, T - (2 << j))
        self.V_ring[:, self.slot(j, torch.arange(p0, T, device=slab.device))] = slab[:, p0:]

    def bind(self, mixer):
        """Per-prefill derived data: the gate readouts transposed once, (L, gh, H) contiguous, so a
        captured step does not copy them on every replay."""
        self.readout_t = [W.transpose(1, 2).contiguous() for W, _ in mixer._gate_params()]

    def advance(self, mx, h, pos):
        """One position through the mixer at device position pos ((1,) int64): records B_hist[pos],
        rg_hist[pos] and the ring slots of pos at every level; returns linear_out of the level-L
        state (reference decoding.py:187-222, fused_step.py:26-88)."""
        Bb = h.shape[0]
        L, H, hd = self.L, self.H, self.hd
        V0, A, B_t = mx.project(h)
        self.B_hist.index_copy_(1, pos, B_t.unsqueeze(1))
        src = pos - self.lags                                        # level-l source position
        live = (src >= 0).to(h.dtype).view(1, L, 1)
        src = src.clamp(min=0)
        hid = F.relu(A.unsqueeze(1) + self.B_hist.index_select(1, src) * live) ** 2      # (B, L, gh)
        pre = [level_gate_matmul(hid.unsqueeze(1), W, W_t)[:, 0] + b
               for (W, b), W_t in zip(mx._gate_params(), self.readout_t)]               # (B, L, H)
        admit, forget, transmit = mx.activate(*pre, live)
        self.rg_hist.index_copy_(1, pos, transmit.unsqueeze(1))
        T_max = self.rg_hist.shape[1]
        r_src = self.rg_hist.view(Bb, T_max * L, H).index_select(1, src * L + self.level_ids)
        V_src = self.V_ring.index_select(1, self.offsets + (src & self.masks)).view(Bb, L, H, hd)
        msg = r_src.unsqueeze(-1) * V_src
        V = V0.view(Bb, H, hd)
        entering = []
        for l in range(L):
            entering.append(V)
            V = mx.level_update(V, forget[:, l].unsqueeze(-1), admit[:, l].unsqueeze(-1), msg[:, l])
        self.V_ring.index_copy_(1, self.offsets + (pos & self.masks),
                                torch.stack(entering, 1).view(Bb, L, H * hd))
        return mx.linear_out(V.reshape(Bb, H * hd))

    def recorder(self, mx, T):
        return _PromptRecorder(self, mx, T)


class _PromptRecorder:
    """Takes, from the mixer's parallel forward over a T-token prompt, what the decoder keeps:
    B_hist rows, transmit gates of every level and the ring slabs (reference decoding.py:143-185).
    Levels at or beyond n_lv = active_levels(L, T) have no source inside the prompt: their state
    passes through unchanged, and their transmit gates are those of a masked source, sigmoid of the
    readout of relu(A)^2."""

    def __init__(self, cache, mx, T):
        self.c, self.mx, self.T = cache, mx, T
        self.n_lv = active_levels(cache.L, T)

    def sources(self, A, B_src):
        c, T = self.c, self.T
        c.B_hist[:, :T] = B_src
        if self.n_lv < c.L:
            hid0 = F.relu(A) ** 2
            W, b = self.mx.reset_out[self.n_lv:], self.mx.reset_out_bias[self.n_lv:]
            pre = F.linear(hid0, W.reshape(-1, W.shape[-1])).unflatten(-1, W.shape[:2]) + b
            c.rg_hist[:, :T, self.n_lv:] = torch.sigmoid(pre)

    def transmit(self, r):                                           # (B*H, T, n_lv)
        c, T = self.c, self.T
        c.rg_hist[:, :T, :self.n_lv] = r.view(-1, c.H, T, self.n_lv).permute(0, 2, 3, 1)

    def entering(self, l, V):                                        # (B*H, T, hd)
        c, T = self.c, self.T
        slab = V.view(-1, c.H, T, c.hd).transpose(1, 2).reshape(-1, T, c.H * c.hd)
        if l < c.L:
            c.write_slab(l, slab)
        if l == self.n_lv:                         # levels n_lv .. L-1 pass the state through
            for j in range(l + 1, c.L):
                c.write_slab(j, slab)


class _AttnCache:
    """Rotated keys and values of one attention layer, head-major (B, H, Tmax, hd) in keys/values,
    and the per-token step that reads the window through a validity mask over the whole cache (a
    shape that stays fixed under graph capture; reference decoding.py:411-435)."""

    def __init__(self, attn, batch, max_len, device, dtype):
        self.keys = torch.zeros(batch, attn.num_heads, max_len, attn.head_dim, device=device, dtype=dtype)
        self.values = torch.zeros_like(self.keys)
        # materialised RoPE tables: graph capture needs stable device tensors to index
        self.rope_cos, self.rope_sin = attn.rope_tables(max_len, device, dtype)
        self.steps = torch.arange(max_len, device=device)

    @property
    def k(self):
        """Keys in the reference's (B, Tmax, H, hd) indexing (a view)."""
        return self.keys.transpose(1, 2)

    @property
    def v(self):
        return self.values.transpose(1, 2)

    def recorder(self, at, T):
        return self

    def keys_values(self, k, v):                                     # prompt: (B, H, T, hd)
        T = k.shape[2]
        self.keys[:, :, :T] = k
        self.values[:, :, :T] = v

    def advance(self, at, h, pos):
        Bb, H, hd = h.shape[0], at.num_heads, at.head_dim
        cos, sin = self.rope_cos.index_select(0, pos), self.rope_sin.index_select(0, pos)
        q = rope_rotate(at.linear_q(h).view(Bb, H, hd), cos, sin)
        self.keys.index_copy_(2, pos, rope_rotate(at.linear_k(h).view(Bb, H, hd), cos, sin).unsqueeze(2))
        self.values.index_copy_(2, pos, at.linear_v(h).view(Bb, H, hd).unsqueeze(2))
        seen = self.steps <= pos
        if at.window > 0:
            seen &= self.steps > pos - at.window
        scores = torch.matmul(self.keys, q.unsqueeze(-1)).squeeze(-1) / math.sqrt(hd)     # (B, H, Tmax)
        p = torch.softmax(scores.masked_fill(~seen, float("-inf")).float(), dim=-1).to(h.dtype)
        y = torch.matmul(p.unsqueeze(2), self.values).squeeze(2)
        return at.linear_out(y.reshape(Bb, H * hd))


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
        self.pos = torch.zeros(1, dtype=torch.long, device=self.device)

    def _alloc(self, batch):
        if self.caches is None or self.batch != batch:
            self.batch = batch
            self.caches = [
                _AttnCache(blk.attn, batch, self.max_len, self.device, self.dtype)
                if isinstance(blk, AttentionBlock) else
                _TreeLayerCache(blk.mixer, batch, self.max_len, self.device, self.dtype)
                for blk in self.m.blocks]
        for blk, cache in zip(self.m.blocks, self.caches):
            if not isinstance(blk, AttentionBlock):
                cache.bind(blk.mixer)

    def _prefill_layer(self, blk, cache, x, mask):
        """One layer of the parallel forward over the prompt, its state recorded into `cache`."""
        h = blk.norm1(x)
        T = x.shape[1]
        if isinstance(blk, AttentionBlock):
            y = blk.attn._forward_eager(h, record=cache.recorder(blk.attn, T))
        else:
            mx = blk.mixer
            y = mx._forward_eager(h, mask, active_levels(mx.levels, T), record=cache.recorder(mx, T))
        x = x + y
        return x + blk.ffn(blk.norm2(x))

    def _advance(self, tokens, pos):
        """Logits (B, vocab) of `tokens` at device position pos, every layer's state advanced."""
        x = self.m.embedding(tokens).to(self.dtype)
        for blk, cache in zip(self.m.blocks, self.caches):
            layer = blk.attn if isinstance(blk, AttentionBlock) else blk.mixer
            x = x + cache.advance(layer, blk.norm1(x), pos)
            x = x + blk.ffn(blk.norm2(x))
        return self.m.lm_head(self.m.norm_out(x))

    @torch.no_grad()
    def prefill(self, idx):
        """idx: (T,) or (B, T) token ids. Returns (T, vocab) or (B, T, vocab) logits."""
        self._squeeze = idx.dim() == 1
        ids = idx.view(1, -1) if self._squeeze else idx
        _check_single_document(self.m, ids)
        T = ids.shape[1]
        if T > self.max_len:
            raise ValueError(f"prompt of {T} exceeds max_len {self.max_len}")
        self._alloc(ids.shape[0])
        mask = self.m.level_mask(T, ids.device, self.dtype)           # the wrap mask only
        x = self.m.embedding(ids).to(self.dtype)
        for blk, cache in zip(self.m.blocks, self.caches):
            x = self._prefill_layer(blk, cache, x, mask)
        self.t = T
        out = self.m.lm_head(self.m.norm_out(x))
        return out[0] if self._squeeze else out

    @torch.no_grad()
    def step(self, tokens):
        """tokens: scalar, (1,) or (B,). Returns (vocab,) or (B, vocab) logits."""
        if self.t >= self.max_len:
            raise ValueError(f"context exhausted at max_len {self.max_len}")
        toks = tokens.view(-1)
        if toks.shape[0] != self.batch and not (self.batch == 1 and toks.shape[0] == 1):
            raise ValueError(f"got {toks.shape[0]} tokens for batch {self.batch}")
        self.pos.fill_(self.t)
        out = self._advance(toks, self.pos)
        self.t += 1
        return out[0] if self._squeeze else out


class _FusedPrefillDecoder(IncrementalDecoder):
    """The fused decoder's prefill: each tree layer runs the parallel gfx950 kernels -- activated
    gates of all L levels in one launch, the level scan over the active levels in a second, which
    also stores the ring slabs -- and fills the same state (B_hist, rg_hist for every level,
    V_ring; reference decoding.py:143-185). Attention layers (bf16, head width 32/64/128) run the
    banded-attention kernel, which also writes the rotated keys and the values into the caches."""

    def _prefill_layer(self, blk, cache, x, mask):
        from . import fused_attention as fa
        from .fused_gates import input_projections, prefill_gate_scan
        T = x.shape[1]
        h = blk.norm1(x)
        if isinstance(blk, AttentionBlock):
            at = blk.attn
            if not (fa.supported(x.dtype, at.head_dim) and cache.keys.dtype == x.dtype):
                return super()._prefill_layer(blk, cache, x, mask)
            cos, sin = at.rope_tables(T, x.device, x.dtype)
            y = fa.window_attention(at.linear_q(h), at.linear_k(h), at.linear_v(h), cos, sin, at.num_heads,
                                    at.band(T), k_cache=cache.keys, v_cache=cache.values)
            y = at.linear_out(y)
        else:
            mx = blk.mixer
            dt = cache.V_ring.dtype
            V0, A, Bs = input_projections(h, mx)
            cache.B_hist[:, :T] = Bs
            (Wi, bi), (Wf, bf), (Wr, br) = mx._gate_params()
            V = prefill_gate_scan(A.to(dt), Bs.to(dt), Wi, Wf, Wr, bi, bf, br, V0.to(dt), cache.H,
                                  cache.rg_hist, cache.V_ring)
            y = mx.linear_out(V.to(x.dtype))
        x = x + y
        return x + blk.ffn(blk.norm2(x))


class GraphedHybridDecoder:
    """The eager decoder's step recorded once into a HIP graph after the prefill and replayed per
    token; the position lives on the device (t_buf) and the replay advances it."""

    _prefill_cls = IncrementalDecoder

    def __init__(self, model, max_len=None, dtype=None):
        if not torch.cuda.is_available():
            raise RuntimeError(f"{type(self).__name__} requires a GPU")
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
        dev = self.inner.device
        Bb = self.inner.batch
        self.token_buf = torch.zeros(Bb, dtype=torch.long, device=dev)
        self.t_buf = torch.full((1,), self.t, dtype=torch.long, device=dev)
        # rows padded to a multiple of 8 elements: every row starts 16-byte aligned (the released
        # vocabulary, 50257, would leave every odd row 2 bytes off, which costs the sampler's 16-byte
        # row loads ~50%: 26 vs 18 us per launch)
        V = self.m.lm_head.out_features
        self._logits_rows = torch.zeros(Bb, -(-V // 8) * 8, device=dev, dtype=self.dtype)
        self.logits_out = self._logits_rows[:, :V]
        self._prepare()
        self.graph = self._capture(self._step_all)
        return out

    def _prepare(self):
        """Buffers of the captured step (subclasses); runs after each prefill, before capture."""

    def _step_all(self):
        """The captured step: logits of token_buf at t_buf, then t_buf + 1."""
        self.logits_out.copy_(self.inner._advance(self.token_buf, self.t_buf))
        self.t_buf.add_(1)

    def _capture(self, fn):
        """Record fn() into a new HIP graph and return it. fn first runs twice on a side stream so
        allocator pools and library workspaces exist before capture; each warm-up's device position
        advance and any token it wrote are undone afterwards."""
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        token0 = self.token_buf.clone()
        with torch.cuda.stream(side):
            for _ in range(2):
                fn()
                self.t_buf.fill_(self.t)
                self.token_buf.copy_(token0)
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            fn()
        return graph

    @torch.no_grad()
    def step(self, tokens):
        if self.t >= self.max_len:
            raise ValueError(f"context exhausted at max_len {self.max_len}")
        self.token_buf.copy_(tokens.view(-1))
        self.graph.replay()
        self.t += 1
        # the next replay overwrites logits_out: return a copy
        out = self.logits_out.clone()
        return out[0] if self._squeeze else out


class FusedGraphedHybridDecoder(GraphedHybridDecoder):
    """Graphed decoder on gfx950 kernels. Prefill: the parallel gate kernels fill the tree state
    (_FusedPrefillDecoder). Step: per tree layer five launches

        dh_decode_gemv       RMSNorm1 + [W_in; W1x; W1s] -> V0, A, B_hist[t]
        mixer step           batch 1: dh_decode_gates (gate readouts of all L levels, one wave per
                             (level, head)) + dh_decode_scan_out (the level recurrence over the rings
                             inside the linear_out + residual launch); batch > 1:
                             dh_decode_mixer_step (gates and recurrence, one workgroup per (head,
                             block of rows)) + dh_decode_gemv (linear_out + residual)
        dh_decode_gemv       RMSNorm2 + [W_gate; W_up] + SwiGLU
        dh_decode_gemv       linear_down + residual

    in place of ~17 torch ops, the embedding gather folded into the first launch and RMSNorm_out +
    lm_head as one launch. An attention layer is the same chain with dh_decode_gemv for its
    projections and one dh_decode_attention launch (RoPE, cache write, windowed softmax, value
    average) in place of the mixer. Same caches, same graph harness; raises ImportError when the
    kernel library is missing.
    """

    _prefill_cls = _FusedPrefillDecoder
    # (row, head) pairs up to which each head's attention window is split over several workgroups
    # (dh_decode_attention_split + a combine launch) instead of one workgroup per pair
    attn_split_pairs = 64

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
        # the feed-forward's hidden row, written by the up launch and read only by the down launch:
        # on the batched matrix-core path it is kept in MFMA fragment order, (16, ff) whatever the batch
        ff = cfg.dim_feedforward
        self._ffn_frag = (dt == torch.bfloat16 and 2 <= Bb <= 16 and ff % 32 == 0 and ff <= 4096
                          and cfg.d_model % 32 == 0 and cfg.d_model <= 2048)
        self.h_buf = torch.zeros(16, ff, device=dev, dtype=dt) if self._ffn_frag else z(ff)
        self.q_buf, self.k_buf, self.v_buf = z(cfg.d_model), z(cfg.d_model), z(cfg.d_model)
        # staging of the two-launch mixer step, shared by every tree layer (same shapes)
        self.stage = torch.zeros(self._fused_step.stage_floats(Bb, mix0.num_heads, mix0.levels,
                                                               mix0.head_dim), device=dev)
        # small batches split each head's attention window over several workgroups
        # greedy decoding on the device: the step's vocabulary head also writes argmax candidates
        # (batch 1) and a second graph ends with the pick, which becomes the next step's input
        self._greedy_graph = None
        self._greedy_capture = False
        # sampled decoding on the device: a third graph ends with the top-k sampler (its settings
        # are part of the recorded launch, so a change of settings records it again)
        self._sample_graph = None
        self._sample_cfg = None
        self._sample_capture = None
        self.tok_hist = torch.zeros(Bb, self.max_len + 1, dtype=torch.long, device=dev)
        # the greedy pick's candidates at batch > 1: owned by this decoder for the captured graph's
        # lifetime (a shared buffer could be replaced, and freed, under a graph that writes it)
        self.argmax_ws = self._fused_step.argmax_workspace(Bb, self.logits_out.shape[1], dev)
        self.cand = None
        if Bb == 1:
            self.cand = self._fused_step.candidate_buffer(dt, self.logits_out.shape[1], cfg.d_model, 1, dev)
        att0 = next((b.attn for b in self.m.blocks if isinstance(b, AttentionBlock)), None)
        self.attn_ws = None
        if att0 is not None and Bb * att0.num_heads <= self.attn_split_pairs:
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
                w[6], w[7], w[8], w[9] = cache.keys, cache.values, cache.rope_cos, cache.rope_sin
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

    def _persistent_step(self, trace=None):
        p = self._pers
        self._fused_step.persistent_step(p["table"], p["kinds"], p["emb"], p["norm_out"], p["eps"], p["dims"],
                                         self.t_buf, self.token_buf, self.tok_hist, self.logits_out, p["scratch"],
                                         trace=trace)

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
        fr = self._ffn_frag
        fs.decode_gemv(self.x_buf, [(f.linear_gate.weight, self.h_buf, ff, 0),
                                    (f.linear_up.weight, self.h_buf, ff, 0)], self.t_buf,
                       norm_weight=blk.norm2.weight, eps=self._eps(blk.norm2, self.dtype), swiglu=True,
                       frag_out=fr)
        h = self.h_buf[:self.x_buf.shape[0]] if fr else self.h_buf   # B rows for the launch's batch size
        fs.decode_gemv(h, [(f.linear_down.weight, self.x_buf, d, 0)], self.t_buf, resid=self.x_buf, frag_in=fr)

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
            # batch > 1: gate readouts and recurrence as one launch per layer (one workgroup per
            # head and block of rows; 8.1 -> 7.1 us per layer at batch 16 against the two-launch form)
            fs.decode_mixer_step(*gate_args[:-1])
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
                            cache.keys, cache.values, self.t_buf, self.y_buf, at.window, workspace=self.attn_ws)
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
        fs.decode_gemv(self.x_buf, [(self.m.lm_head.weight, self.logits_out, self.logits_out.stride(0), 0)], self.t_buf,
                       norm_weight=self.m.norm_out.weight, eps=self._eps(self.m.norm_out, self.dtype),
                       t_advance=self.t_buf, argmax_cand=cand)
        if self._greedy_capture:
            # greedy pick into the next step's token input and the token history (at the new position)
            if cand is not None:
                fs.argmax_reduce(cand, self.token_buf, self.t_buf, self.tok_hist)
            else:
                fs.argmax_tokens(self.logits_out, out=self.token_buf, workspace=self.argmax_ws)
                self.tok_hist.index_copy_(1, self.t_buf, self.token_buf.unsqueeze(1))
        elif self._sample_capture is not None:
            # sampled pick (draws keyed by the new position) into token_buf and the token history
            temperature, top_k, seed = self._sample_capture
            fs.sample_tokens(self.logits_out, temperature, top_k, seed, self.t_buf, out=self.token_buf,
                             hist=self.tok_hist)

    @torch.no_grad()
    def greedy_start(self, logits):
        """Start device-side greedy decoding after prefill: the argmax of `logits` (the prefill's
        last-position logits, (B, V) or (V,)) becomes the token fed to the next step and the first
        entry of tok_hist (at the current position)."""
        lg = logits.view(-1, logits.shape[-1])
        self._fused_step.argmax_tokens(lg, out=self.token_buf, workspace=self.argmax_ws)
        self.tok_hist[:, self.t] = self.token_buf

    @torch.no_grad()
    def sample_start(self, logits, temperature=1.0, top_k=None, seed=0):
        """Start device-side sampled decoding after prefill: temperature / top-k sampling
        (fused_step.sample_tokens: Philox draws keyed by `seed`, the device position and the row) of
        `logits` (the prefill's last-position logits) becomes the token fed to the next step and the
        first entry of tok_hist; step_sample() then keeps the same settings. The tokens equal those
        of step() followed by sample_tokens(logits, temperature, top_k, seed, t_buf)."""
        cfg = (float(temperature), top_k, int(seed))
        if cfg != self._sample_cfg:
            self._sample_graph = None
            self._sample_cfg = cfg
        lg = logits.view(-1, logits.shape[-1])
        self._fused_step.sample_tokens(lg, cfg[0], top_k, cfg[2], self.t_buf, out=self.token_buf)
        self.tok_hist[:, self.t] = self.token_buf

    @torch.no_grad()
    def step_sample(self):
        """One decode step fed by the token in token_buf, ending with the sampler of sample_start():
        the next token goes to token_buf and tok_hist[:, t + 1] on the device -- one graph replay per
        token, no host work (the sampling branch of fast_generate)."""
        if self._sample_cfg is None:
            raise RuntimeError("step_sample: call sample_start() first")
        if self.t >= self.max_len:
            raise ValueError(f"context exhausted at max_len {self.max_len}")
        if self._sample_graph is None:
            self._sample_capture = self._sample_cfg
            try:
                self._sample_graph = self._capture(self._step_all)
            finally:
                self._sample_capture = None
        self._sample_graph.replay()
        self.t += 1

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
                self._greedy_graph = self._capture(self._step_all)
            finally:
                self._greedy_capture = False
        self._greedy_graph.replay()
        self.t += 1

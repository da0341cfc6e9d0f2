"""Dispatcher-Hybrid causal LM: dyadic shift-and-sum mixer layers plus a few sliding-window
attention layers.

Host-side module tree with the reference's class names, parameter names and shapes
(reference dispatcher_hybrid/modeling_dispatcher.py:36-442), so released checkpoints load 1:1 and
code written against the reference runs unchanged. The mixer, per layer, for level
l = 0 .. log2(max_len) - 1 (lag 2^l):

    h_l(t) = relu(W1x.x(t) + W1s.x(t - 2^l))^2            gate hidden
    a_l(t) = sigmoid(Wa_l.h_l(t) + b_a)                    admit
    f_l(t) = sigmoid(Wf_l.h_l(t) + b_f)                    forget
    r_l(t) = sigmoid(Wr_l.h_l(t) + b_r)                    transmit (applied at the source)
    V(t)  <- f_l(t) V(t) + a_l(t) (r_l V)(t - 2^l)

Two implementations of the mixer, selected per module by `use_fused_gates`:
  * eager torch ops (the default, identical algebra to the reference's eager branch);
  * the fused path (`model.enable_fused_gates()`): the gate pre-activations and the level scan run
    as two gfx950 HIP kernels (``dh_gate_preacts_fwd``, ``dh_level_scan_fwd``). It needs the GPU
    and the kernel library, and raises instead of falling back when either is missing.
"""

import math
import sys

import torch
import torch.nn as nn
import torch.nn.functional as F
from transformers import PreTrainedModel
from transformers.generation import GenerationMixin
from transformers.modeling_outputs import CausalLMOutput

from .configuration_dispatcher import DispatcherConfig


def active_levels(levels, length):
    """Levels that can reach back inside a length-T sequence: min(L, floor(log2 T) + 1)
    (reference modeling_dispatcher.py:76)."""
    return min(levels, max(int(length), 1).bit_length())


def level_gate_matmul(hidden, W, W_t=None):
    """pre[b,t,l,h] = sum_g hidden[b,t,l,g] * W[l,h,g] for hidden (b,t,n,g), W (n,h,g).

    Batched over levels with both bmm operands contiguous (a transposed right operand to a bf16
    bmm is avoided on purpose). W_t: W already transposed to a contiguous (n, g, h), for callers
    that apply the same readout many times."""
    b, t, n, g = hidden.shape
    lhs = hidden.permute(2, 0, 1, 3).reshape(n, b * t, g)
    rhs = W.transpose(1, 2).contiguous() if W_t is None else W_t
    return torch.bmm(lhs, rhs).view(n, b, t, -1).permute(1, 2, 0, 3)


class DispatcherMixer(nn.Module):
    """Gated dyadic shift-and-sum sequence mixer (the layer that replaces attention)."""

    def __init__(self, config: DispatcherConfig):
        super().__init__()
        d, H = config.d_model, config.num_heads
        self.embed_dim = d
        self.num_heads = H
        self.head_dim = d // H
        self.levels = config.levels
        self.shifts = [1 << l for l in range(self.levels)]
        self.use_fused_gates = False
        gh = d                                              # gate hidden width of the release
        self.linear_in = nn.Linear(d, d, bias=False)
        self.gate_hidden = nn.Linear(d, gh, bias=False)     # W1x (destination)
        self.gate_hidden_src = nn.Linear(d, gh, bias=False) # W1s (source)
        L = self.levels
        self.gate_out = nn.Parameter(torch.empty(L, H, gh))
        self.gate_out_bias = nn.Parameter(torch.full((L, H), float(config.gate_bias_flat)))
        self.forget_out = nn.Parameter(torch.empty(L, H, gh))
        self.forget_out_bias = nn.Parameter(torch.full((L, H), float(config.gate_fbias_flat)))
        self.reset_out = nn.Parameter(torch.empty(L, H, gh))
        self.reset_out_bias = nn.Parameter(torch.full((L, H), 2.0))
        self.linear_out = nn.Linear(d, d, bias=False)

    def _gate_params(self):
        return ((self.gate_out, self.gate_out_bias), (self.forget_out, self.forget_out_bias),
                (self.reset_out, self.reset_out_bias))

    def project(self, h):
        """The three input projections of a normalised input h (..., d): V0 = W_in.h (the state
        entering level 0), A = W1x.h (destination half of the gate hidden), B = W1s.h (source half,
        read again 2^l positions later)."""
        return self.linear_in(h), self.gate_hidden(h), self.gate_hidden_src(h)

    @staticmethod
    def activate(pre_i, pre_f, pre_r, m):
        """Gate heads from pre-activations under the edge mask m (1: level live, 0: no source):
        admit = sigmoid(pre_i) m, forget = sigmoid(pre_f) m + 1 - m (a dead level keeps its state),
        transmit = sigmoid(pre_r), unmasked: it is read at the source, where a dead destination
        already has admit = 0 (reference modeling_dispatcher.py:111-114)."""
        return (torch.sigmoid(pre_i) * m, torch.sigmoid(pre_f) * m + (1.0 - m), torch.sigmoid(pre_r))

    @staticmethod
    def level_update(V, forget, admit, msg):
        """One level of the recurrence: V <- forget V + admit msg, msg = transmit(src) V(src)
        (reference modeling_dispatcher.py:116-121)."""
        return forget * V + admit * msg

    def forward(self, x, mask):
        """x (B, T, d); mask (T, L) level mask or (B, T, L) level x doc-reset mask."""
        n_lv = active_levels(self.levels, x.shape[1])
        if self.use_fused_gates:
            return self._forward_fused(x, mask, n_lv)
        return self._forward_eager(x, mask, n_lv)

    # -- eager torch path ------------------------------------------------------------------
    def _masks(self, mask, Bb, T, n_lv):
        H = self.num_heads
        lm = mask[..., :n_lv]
        if mask.dim() == 3:
            m_src = lm.unsqueeze(-1)                                         # (B, T, n, 1)
            m_heads = lm.unsqueeze(1).expand(Bb, H, T, n_lv).reshape(Bb * H, T, n_lv)
        else:
            m_src = lm.reshape(1, T, n_lv, 1)
            m_heads = lm
        return m_src, m_heads

    def _scan_eager(self, V, pre_i, pre_f, pre_r, m_heads, Bb, T, n_lv, record=None):
        """Sigmoid heads, masks and the level loop on (B*H, T, hd) V (reference :86-88, :111-121).
        record (optional): told the transmit gates (B*H, T, n_lv) and the state entering every level
        (record.transmit, record.entering) -- what an incremental decoder keeps of a prompt."""
        H = self.num_heads

        def per_head(pre):
            return pre.permute(0, 3, 1, 2).reshape(Bb * H, T, n_lv)

        admit, forget, transmit = (g.to(V.dtype) for g in self.activate(
            per_head(pre_i), per_head(pre_f), per_head(pre_r), m_heads))
        if record is not None:
            record.transmit(transmit)
            record.entering(0, V)
        for l, shift in enumerate(self.shifts[:n_lv]):
            msg = torch.roll(transmit[..., l:l + 1] * V, shifts=shift, dims=1)
            V = self.level_update(V, forget[..., l:l + 1], admit[..., l:l + 1], msg)
            if record is not None:
                record.entering(l + 1, V)
        return V

    def _forward_eager(self, x, mask, n_lv, record=None):
        Bb, T = x.shape[0], x.shape[1]
        H, hd = self.num_heads, self.head_dim
        V0, A, Bs = self.project(x)
        if record is not None:
            record.sources(A, Bs)
        # heads go to the batch axis through a transpose (a plain reshape would tile the sequence)
        V = V0.view(Bb, T, H, hd).transpose(1, 2).reshape(Bb * H, T, hd)
        m_src, m_heads = self._masks(mask, Bb, T, n_lv)
        lagged = torch.stack([torch.roll(Bs, shifts=s, dims=1) for s in self.shifts[:n_lv]], dim=2)
        hidden = F.relu(A.unsqueeze(2) + lagged * m_src) ** 2            # (B, T, n, gh)
        pre_i, pre_f, pre_r = (level_gate_matmul(hidden, W[:n_lv]) + b[:n_lv]
                               for W, b in self._gate_params())
        V = self._scan_eager(V, pre_i, pre_f, pre_r, m_heads, Bb, T, n_lv, record)
        V = V.view(Bb, H, T, hd).transpose(1, 2).reshape(Bb, T, self.embed_dim)
        return self.linear_out(V)

    # -- fused HIP path --------------------------------------------------------------------
    def _forward_fused(self, x, mask, n_lv):
        if not x.is_cuda:
            raise RuntimeError("fused gates are enabled but the input is on the CPU; move the model "
                               "to the GPU or call enable_fused_gates(False)")
        from .fused_gates import fused_gate_preacts, fused_gate_scan, input_projections
        Bb, T = x.shape[0], x.shape[1]
        H, hd = self.num_heads, self.head_dim
        needs_grad = torch.is_grad_enabled() and (
            x.requires_grad or any(p.requires_grad for p in self.parameters()))
        if needs_grad:
            V0, A, Bs = self.linear_in(x), self.gate_hidden(x), self.gate_hidden_src(x)
        else:
            V0, A, Bs = input_projections(x, self)
        m3 = mask[..., :n_lv] if mask.dim() == 3 else None
        (Wi, bi), (Wf, bf), (Wr, br) = self._gate_params()
        if needs_grad:
            # differentiable: the fused pre-activations (custom op with autograd) + torch scan
            pre_i, pre_f, pre_r = fused_gate_preacts(A, Bs, Wi, Wf, Wr, bi, bf, br, n_lv, m3)
            _, m_heads = self._masks(mask, Bb, T, n_lv)
            V = V0.view(Bb, T, H, hd).transpose(1, 2).reshape(Bb * H, T, hd)
            V = self._scan_eager(V, pre_i, pre_f, pre_r, m_heads.to(V.dtype), Bb, T, n_lv)
            V = V.view(Bb, H, T, hd).transpose(1, 2).reshape(Bb, T, self.embed_dim)
        else:
            # inference: activated gates written head-major, then the level scan (two launches)
            V = fused_gate_scan(A, Bs, Wi, Wf, Wr, bi, bf, br, n_lv, m3, V0, H)
            from .fused_gates import OUT_GEMM_MAX_ROWS, project
            return project(V, [self.linear_out], OUT_GEMM_MAX_ROWS)[0]
        return self.linear_out(V)


def rope_rotate(x, cos, sin):
    """Rotate interleaved pairs (x[2i], x[2i+1]) by the angle whose cos/sin are given
    (reference modeling_dispatcher.py:163-166)."""
    pairs = x.unflatten(-1, (-1, 2))
    even, odd = pairs[..., 0], pairs[..., 1]
    return torch.stack((even * cos - odd * sin, even * sin + odd * cos), dim=-1).flatten(-2)


def causal_window_attention(q, k, v, window, block=256):
    """softmax(q k^T / sqrt(hd)) v over keys s with t - window < s <= t (window <= 0: all s <= t).

    q, k, v: (B, H, T, hd). Evaluated in query blocks over just the band of keys each block can
    see, with contiguous operands to every matmul; softmax in fp32.
    """
    Bb, H, T, hd = q.shape
    scale = 1.0 / math.sqrt(hd)
    kT = k.transpose(-2, -1).contiguous()                     # (B, H, hd, T)
    out = torch.empty_like(q)
    for q0 in range(0, T, block):
        q1 = min(T, q0 + block)
        lo = 0 if window <= 0 else max(0, q0 - window + 1)
        s = torch.matmul(q[:, :, q0:q1], kT[..., lo:q1].contiguous()).float() * scale
        tq = torch.arange(q0, q1, device=q.device).unsqueeze(1)
        tk = torch.arange(lo, q1, device=q.device).unsqueeze(0)
        ok = tk <= tq
        if window > 0:
            ok = ok & (tq - tk < window)
        p = torch.softmax(s.masked_fill(~ok, float("-inf")), dim=-1).to(q.dtype)
        out[:, :, q0:q1] = torch.matmul(p, v[:, :, lo:q1].contiguous())
    return out


class WindowAttention(nn.Module):
    """Causal sliding-window multi-head attention with interleaved RoPE."""

    def __init__(self, config: DispatcherConfig):
        super().__init__()
        d, H = config.d_model, config.num_heads
        self.embed_dim = d
        self.num_heads = H
        self.head_dim = d // H
        self.window = config.attn_window
        self.linear_q = nn.Linear(d, d, bias=False)
        self.linear_k = nn.Linear(d, d, bias=False)
        self.linear_v = nn.Linear(d, d, bias=False)
        self.linear_out = nn.Linear(d, d, bias=False)
        self._rope_cache = {}
        self.use_fused = False      # gfx950 banded-attention kernel for inference (enable_fused_gates)

    def rope_tables(self, length, device, dtype):
        """cos/sin of angle t * 10000^(-2i/hd), (length, hd/2), cached per (length, device, dtype)
        -- one entry each, never replaced: a HIP graph captured over a forward keeps reading the
        tables it was captured with. Not a buffer: derived data stays out of checkpoints
        (reference :144-161)."""
        key = (length, device, dtype)
        tables = self._rope_cache.get(key)
        if tables is None:
            inv_freq = torch.pow(10000.0, -torch.arange(0, self.head_dim, 2, device=device,
                                                        dtype=torch.float32) / self.head_dim)
            ang = torch.outer(torch.arange(length, device=device, dtype=torch.float32), inv_freq)
            tables = self._rope_cache[key] = (ang.cos().to(dtype), ang.sin().to(dtype))
        return tables

    def apply_rope(self, x, length):
        cos, sin = self.rope_tables(length, x.device, x.dtype)
        return rope_rotate(x, cos, sin)

    def forward(self, x):
        T = x.shape[1]
        if self.use_fused and not torch.is_grad_enabled() and x.is_cuda:
            from . import fused_attention as fa
            if fa.supported(x.dtype, self.head_dim):
                from .fused_gates import OUT_GEMM_MAX_ROWS, QKV_GEMM_MAX_ROWS, project
                # q, k, v as one GEMM launch (up to QKV_GEMM_MAX_ROWS rows); RoPE, banded scores,
                # softmax and the value average in one launch, (B, T, d) in/out
                q, k, v = project(x, [self.linear_q, self.linear_k, self.linear_v], QKV_GEMM_MAX_ROWS)
                cos, sin = self.rope_tables(T, x.device, x.dtype)
                y = fa.window_attention(q, k, v, cos, sin, self.num_heads, self.band(T))
                return project(y, [self.linear_out], OUT_GEMM_MAX_ROWS)[0]
        return self._forward_eager(x)

    def band(self, T):
        """The window a length-T sequence sees; 0 when it covers the whole sequence."""
        return self.window if 0 < self.window < T else 0

    def _forward_eager(self, x, record=None):
        """record (optional): told the rotated keys and the values, (B, H, T, hd) -- what an
        incremental decoder keeps of a prompt."""
        Bb, T = x.shape[0], x.shape[1]
        shape = (Bb, T, self.num_heads, self.head_dim)
        q = self.apply_rope(self.linear_q(x).view(shape).transpose(1, 2), T)
        k = self.apply_rope(self.linear_k(x).view(shape).transpose(1, 2), T)
        v = self.linear_v(x).view(shape).transpose(1, 2)
        if record is not None:
            record.keys_values(k, v)
        y = causal_window_attention(q, k, v, self.band(T))
        return self.linear_out(y.transpose(1, 2).reshape(Bb, T, self.embed_dim))


class SwiGLU(nn.Module):
    """linear_down(silu(linear_gate(h)) * linear_up(h)) (reference modeling_dispatcher.py:188-197).
    With use_fused (set by enable_fused_gates) and no autograd, bf16 layers run linear_gate,
    linear_up and the activation as one dh_proj_gemm_swiglu launch (the two GEMM outputs never
    reach memory), other fp32/bf16 layers the two GEMMs and one dh_silu_mul launch; both at the
    eager rounding points. In bf16, linear_down runs on dh_proj_gemm up to DOWN_GEMM_MAX_ROWS rows."""

    use_fused = False

    def __init__(self, config: DispatcherConfig):
        super().__init__()
        d, ff = config.d_model, config.dim_feedforward
        self.linear_gate = nn.Linear(d, ff, bias=False)
        self.linear_up = nn.Linear(d, ff, bias=False)
        self.linear_down = nn.Linear(ff, d, bias=False)

    def forward(self, h):
        if (self.use_fused and h.is_cuda and not torch.is_grad_enabled()
                and h.dtype in (torch.float32, torch.bfloat16)):                   # dh_silu_mul's dtypes
            from .fused_gates import DOWN_GEMM_MAX_ROWS, fused_swiglu, project, silu_mul, swiglu_fits
            if swiglu_fits(h, self.linear_gate, self.linear_up):
                a = fused_swiglu(h, self.linear_gate.weight, self.linear_up.weight)
            else:
                g = self.linear_gate(h)
                a = silu_mul(g, self.linear_up(h), out=g)
            # (bf16: the shapes it was measured on; fp32 stays on the library)
            return project(a, [self.linear_down], DOWN_GEMM_MAX_ROWS if a.dtype == torch.bfloat16 else 0)[0]
        return self.linear_down(F.silu(self.linear_gate(h)) * self.linear_up(h))


class DispatcherBlock(nn.Module):
    """Pre-norm residual block: mixer, then SwiGLU."""

    def __init__(self, config: DispatcherConfig):
        super().__init__()
        self.mixer = DispatcherMixer(config)
        self.ffn = SwiGLU(config)
        self.norm1 = nn.RMSNorm(config.d_model)
        self.norm2 = nn.RMSNorm(config.d_model)

    def forward(self, x, mask):
        x = x + self.mixer(self.norm1(x), mask)
        return x + self.ffn(self.norm2(x))


class AttentionBlock(nn.Module):
    """Pre-norm residual block: sliding-window attention (ignores the mixer mask), then SwiGLU."""

    def __init__(self, config: DispatcherConfig):
        super().__init__()
        self.attn = WindowAttention(config)
        self.ffn = SwiGLU(config)
        self.norm1 = nn.RMSNorm(config.d_model)
        self.norm2 = nn.RMSNorm(config.d_model)

    def forward(self, x, mask=None):
        x = x + self.attn(self.norm1(x))
        return x + self.ffn(self.norm2(x))


class DispatcherPreTrainedModel(PreTrainedModel):
    config_class = DispatcherConfig
    base_model_prefix = "dispatcher"
    supports_gradient_checkpointing = True
    _no_split_modules = ["DispatcherBlock", "AttentionBlock"]

    def _init_weights(self, module):
        # N(0, 0.02) for every projection, embedding and gate readout; W1s (gate_hidden_src)
        # starts at zero (reference modeling_dispatcher.py:236-247).
        if isinstance(module, (nn.Linear, nn.Embedding)):
            nn.init.normal_(module.weight, mean=0.0, std=0.02)
        elif isinstance(module, DispatcherMixer):
            for p in (module.gate_out, module.forget_out, module.reset_out):
                nn.init.normal_(p, mean=0.0, std=0.02)
            with torch.no_grad():
                module.gate_hidden_src.weight.zero_()


class DispatcherHybridForCausalLM(DispatcherPreTrainedModel, GenerationMixin):
    """Dispatcher / sliding-window-attention hybrid causal language model.

    `generate()` recomputes the prefix each step; `fast_generate()` uses the incremental decoders
    of `dispatcher_hybrid.decoding` (per-token cost flat in context).
    """

    _tied_weights_keys = {"lm_head.weight": "embedding.weight"}
    main_input_name = "input_ids"

    def __init__(self, config: DispatcherConfig):
        super().__init__(config)
        attn_slots = set(config.attn_layers) if config.attn_window > 0 else set()
        self.embedding = nn.Embedding(config.vocab_size, config.d_model)
        self.blocks = nn.ModuleList(
            AttentionBlock(config) if (i + 1) in attn_slots else DispatcherBlock(config)
            for i in range(config.num_layers))
        self.norm_out = nn.RMSNorm(config.d_model)
        self.lm_head = nn.Linear(config.d_model, config.vocab_size, bias=False)
        self._mask_cache = {}
        self._src_cache = {}
        self.post_init()

    def level_mask(self, length, device=None, dtype=torch.float32):
        """mask[t, l] = 1 iff position t has a predecessor 2^l back (t >= 2^l), (T, L).
        This is what keeps roll()'s wrapped (future) rows out of the eager mixer."""
        key = (length, device, dtype)
        mask = self._mask_cache.get(key)
        if mask is None:                  # one entry per key, never replaced (see WindowAttention.rope_tables)
            t = torch.arange(length, device=device).unsqueeze(1)
            lag = torch.tensor([1 << l for l in range(self.config.levels)], device=device)
            mask = self._mask_cache[key] = ((t >= lag) & (lag < length)).to(dtype)
        return mask

    def get_input_embeddings(self):
        return self.embedding

    def set_input_embeddings(self, value):
        self.embedding = value

    def get_output_embeddings(self):
        return self.lm_head

    def set_output_embeddings(self, value):
        self.lm_head = value

    def _tree_mask(self, input_ids, length):
        """Level mask, times (doc_reset) "source and destination are in the same document".

        doc(t) counts the EOTs strictly before t, so an EOT belongs to the document it ends;
        level l's edge t <- t-2^l (index taken mod T, as roll() does) is kept iff the two doc ids
        match (reference modeling_dispatcher.py:311-323)."""
        dtype = self.embedding.weight.dtype
        if (self.config.doc_reset and getattr(self, "_fused_norms", False) and input_ids.is_cuda
                and input_ids.dtype == torch.int64 and dtype in (torch.float32, torch.bfloat16)):
            from .fused_gates import TREE_MASK_MAX_LEN, TREE_MASK_MAX_LEVELS, TREE_MASK_MAX_ROWS, tree_mask
            if (length <= TREE_MASK_MAX_LEN and 1 <= self.config.levels <= TREE_MASK_MAX_LEVELS
                    and input_ids.shape[0] <= TREE_MASK_MAX_ROWS):
                # the same 0/1 values in one launch (dh_tree_mask) instead of the eight below
                return tree_mask(input_ids, self.config.levels, self.config.eot_token, dtype)
        mask = self.level_mask(length, input_ids.device, dtype)
        if not self.config.doc_reset:
            return mask
        is_eot = (input_ids == self.config.eot_token).to(mask.dtype)
        doc = torch.cumsum(is_eot, dim=1) - is_eot
        # every level's source index (t - 2^l) mod T in one (T, L) table (cached with the level mask),
        # so the comparison is one gather instead of a few launches per level
        src = self._src_index(length, input_ids.device)
        same = (doc.unsqueeze(-1) == doc[:, src]).to(mask.dtype)
        return mask.unsqueeze(0) * same[..., :mask.shape[-1]]

    def _src_index(self, length, device):
        key = (length, device)
        src = self._src_cache.get(key)
        if src is None:
            t = torch.arange(length, device=device).unsqueeze(1)
            lag = torch.tensor([1 << l for l in range(self.config.levels)], device=device)
            src = self._src_cache[key] = (t - lag) % length
        return src

    def forward(self, input_ids=None, attention_mask=None, labels=None, inputs_embeds=None,
                use_cache=None, output_attentions=None, output_hidden_states=None,
                return_dict=None, **kwargs):
        if input_ids is None:
            raise ValueError("DispatcherHybridForCausalLM requires input_ids "
                             "(the tree mask is built from token identities)")
        return_dict = True if return_dict is None else return_dict
        length = input_ids.size(1)
        if length > self.config.max_len:
            raise ValueError(f"sequence length {length} exceeds max_len {self.config.max_len}")
        mask = self._tree_mask(input_ids, length)
        hidden_states = () if output_hidden_states else None
        x = self.embedding(input_ids)
        if self._fused_norm_ok(x, output_hidden_states):
            x = self._blocks_fused_norms(x, mask)
        else:
            for block in self.blocks:
                if output_hidden_states:
                    hidden_states = hidden_states + (x,)
                if getattr(self, "gradient_checkpointing", False) and self.training:
                    x = self._gradient_checkpointing_func(block.__call__, x, mask)
                else:
                    x = block(x, mask)
            x = self.norm_out(x)
        if output_hidden_states:
            hidden_states = hidden_states + (x,)
        logits = self.lm_head(x)
        loss = None
        if labels is not None:
            loss = F.cross_entropy(logits[:, :-1].reshape(-1, logits.size(-1)),
                                   labels[:, 1:].reshape(-1))
        if not return_dict:
            return (loss, logits) if loss is not None else (logits,)
        return CausalLMOutput(loss=loss, logits=logits, hidden_states=hidden_states)

    def prepare_inputs_for_generation(self, input_ids, **kwargs):
        return {"input_ids": input_ids[:, -self.config.max_len:]}

    def _fused_norm_ok(self, x, output_hidden_states):
        """Whether the block loop may fuse each residual add with the RMSNorm after it: inference on
        the GPU, weighted norms in x's dtype, and a width dh_add_rmsnorm takes (otherwise the
        block-by-block loop runs)."""
        if not (getattr(self, "_fused_norms", False) and x.is_cuda and not torch.is_grad_enabled()
                and not output_hidden_states and x.dtype in (torch.float32, torch.bfloat16) and len(self.blocks)):
            return False
        from .fused_gates import add_rmsnorm_fits
        if not add_rmsnorm_fits(x.shape[-1], x.dtype):
            return False
        norms = [self.norm_out] + [n for blk in self.blocks for n in (blk.norm1, blk.norm2)]
        return all(n.weight is not None and n.weight.dtype == x.dtype and tuple(n.normalized_shape) == (x.shape[-1],)
                   for n in norms)

    def _blocks_fused_norms(self, x, mask):
        """The blocks and norm_out with every residual add fused into the RMSNorm that follows it
        (dh_add_rmsnorm): norm1 of the first block, then per block sublayer -> add + norm2 ->
        SwiGLU -> add + the next block's norm1 (norm_out after the last). Same sums as the
        block-by-block loop, bf16-rounded at the same points; returns norm_out's output."""
        from .fused_gates import add_rmsnorm
        blocks = list(self.blocks)
        h = blocks[0].norm1(x)
        x = x.contiguous()
        for i, blk in enumerate(blocks):
            y = blk.attn(h) if hasattr(blk, "attn") else blk.mixer(h, mask)
            x, h = add_rmsnorm(x, y, blk.norm2, out=x)
            y = blk.ffn(h)
            nxt = blocks[i + 1].norm1 if i + 1 < len(blocks) else self.norm_out
            x, h = add_rmsnorm(x, y, nxt, out=x)
        return h

    def enable_fused_gates(self, enabled=True):
        """Run every mixer's gate pipeline and level scan on the gfx950 HIP kernels (and, without
        autograd, every SwiGLU activation on dh_silu_mul, every residual add and the RMSNorm after
        it on dh_add_rmsnorm and, in bf16, every attention layer on the banded-attention kernel).

        Loads the kernel library now (raising ImportError if it is missing) rather than in the
        middle of a forward. The fused path needs GPU tensors; returns self.
        """
        if enabled:
            from . import fused_attention, fused_gates  # noqa: F401  (fail now, not mid-forward)
        for blk in self.blocks:
            if hasattr(blk, "mixer"):
                blk.mixer.use_fused_gates = bool(enabled)
            if hasattr(blk, "attn"):
                # inference only: attention layers take the banded-attention kernel (bf16)
                blk.attn.use_fused = bool(enabled)
            if hasattr(blk, "ffn"):
                # inference only: the SwiGLU activation in one launch
                blk.ffn.use_fused = bool(enabled)
        # inference only: each residual add fused with the RMSNorm after it
        self._fused_norms = bool(enabled)
        return self

    @torch.no_grad()
    def graphed_logits(self, input_ids):
        """Logits of the forward through a HIP graph captured once per input shape and device: a
        static-shape prefill, one graph replay instead of the forward's several hundred launches
        issued from the host (the C2 forward: 2.8 vs 5.6 ms on MI355X).

        The first call for a shape runs two warm-up forwards on a side stream and captures one
        forward; every call copies input_ids into the graph's input buffer and replays. The result
        is the graph's output buffer: the next call with the same shape overwrites it (clone it to
        keep it). The parameters must stay where they are between calls; in-place updates of the
        weights are seen, but the fused path reads bf16 gate biases through fp32 copies made when a
        forward runs, so after changing those call release_graphs() to capture again. The path
        captured is the one active at the first call, so call enable_fused_gates() first for the
        fused kernels. Bit for bit equal to self(input_ids).logits on that path.
        """
        if not input_ids.is_cuda:
            raise ValueError("graphed_logits needs input_ids on a GPU")
        key = (tuple(input_ids.shape), input_ids.dtype, input_ids.device)
        graphs = self.__dict__.setdefault("_forward_graphs", {})
        entry = graphs.get(key)
        if entry is None:
            static_ids = input_ids.clone()
            side = torch.cuda.Stream(device=input_ids.device)
            side.wait_stream(torch.cuda.current_stream(input_ids.device))
            with torch.cuda.stream(side):
                for _ in range(2):
                    self(static_ids)
            torch.cuda.current_stream(input_ids.device).wait_stream(side)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                out = self(static_ids).logits
            # the graph reads the fp32 gate-bias copies made by the warm-up forwards: keep them alive
            # even if a later forward replaces them (after a bias update)
            fg = sys.modules.get(__package__ + ".fused_gates")
            keep = [e[3] for e in getattr(fg, "_BIAS_F32", {}).values()]
            entry = graphs[key] = (graph, static_ids, out, keep)
        graph, static_ids, out, _ = entry
        static_ids.copy_(input_ids)
        graph.replay()
        return out

    def release_graphs(self):
        """Drop the forward graphs captured by graphed_logits (and their buffers)."""
        self.__dict__.pop("_forward_graphs", None)

    @torch.no_grad()
    def fast_generate(self, input_ids, max_new_tokens=50, do_sample=False, temperature=1.0,
                      top_k=None, eos_token_id=None, num_return_sequences=1, decoder="auto"):
        """Generate with an incremental decoder (per-token cost O(log t), flat in context).

        input_ids (T,) or (B, T): rows advance in lockstep, so a batch shares one prompt length.
        num_return_sequences tiles one prompt into that many sampled rows. decoder: "auto"
        (fused -> graphed -> eager on GPU, eager on CPU), "eager", "graphed" (HIP graph) or
        "fused" (HIP graph + gfx950 mixer kernels). Rows that emit eos are frozen at eos.
        Returns (B, T + generated) ids including the prompt (reference :379-442).
        """
        from .decoding import FusedGraphedHybridDecoder, GraphedHybridDecoder, IncrementalDecoder

        ids = input_ids.view(1, -1) if input_ids.dim() == 1 else input_ids
        if num_return_sequences > 1:
            if ids.shape[0] != 1:
                raise ValueError("num_return_sequences needs a single prompt")
            if not do_sample:
                raise ValueError("num_return_sequences without sampling would return identical rows")
            ids = ids.expand(num_return_sequences, -1)
        choices = {"eager": IncrementalDecoder, "graphed": GraphedHybridDecoder,
                   "fused": FusedGraphedHybridDecoder}
        if decoder == "auto":
            dec = None
            for name in (["fused", "graphed", "eager"] if ids.is_cuda else ["eager"]):
                try:
                    dec = choices[name](self)
                    break
                except Exception:
                    continue
            if dec is None:
                raise RuntimeError("no usable decoder")
        else:
            if decoder not in choices:
                raise ValueError(f"unknown decoder {decoder!r}; use one of auto, {', '.join(choices)}")
            dec = choices[decoder](self)

        Bb = ids.shape[0]
        logits = dec.prefill(ids)[:, -1]                     # ids is 2-D: (B, T, V) -> (B, V)
        if isinstance(dec, FusedGraphedHybridDecoder) and eos_token_id is None:
            # without eos every pick stays on the device (the last launches of the graphed step); the
            # loop below appends min(max_new_tokens, max_len - t + 1) tokens, the same count here.
            # Sampling: draws keyed by a seed from torch's generator and the device position, the
            # same tokens as the loop's sample_tokens picks
            n = min(max_new_tokens, dec.max_len - dec.t + 1)
            if n <= 0:
                return ids
            t0 = dec.t
            if do_sample:
                seed = int(torch.randint(0, 2 ** 62, (1,)).item())
                dec.sample_start(logits, max(temperature, 1e-6), top_k, seed)
                for _ in range(n - 1):
                    dec.step_sample()
            else:
                dec.greedy_start(logits)
                for _ in range(n - 1):
                    dec.step_greedy()
                dec.check_persistent()                     # a one-launch step that timed out is redone
            return torch.cat([ids, dec.tok_hist[:, t0:t0 + n]], dim=1)
        finished = torch.zeros(Bb, dtype=torch.bool, device=ids.device)
        out = [ids]
        # Through the fused decoder the next token is picked on the device. Greedy: the argmax
        # kernel (a positive temperature and top-k masking never move the maximum, so the tokens
        # are the same). Sampling: the top-k sampler, its draws keyed by a seed taken from torch's
        # generator (torch.manual_seed reproduces a run) and the decoder's device position; the
        # stream of draws is not torch.multinomial's.
        device_pick = None
        if isinstance(dec, FusedGraphedHybridDecoder):
            fs = dec._fused_step
            if not do_sample:
                device_pick = fs.argmax_tokens
            else:
                seed = int(torch.randint(0, 2 ** 62, (1,)).item())
                temp = max(temperature, 1e-6)
                device_pick = lambda lg: fs.sample_tokens(lg, temp, top_k, seed, dec.t_buf)
        for _ in range(max_new_tokens):
            if device_pick is not None:
                nxt = device_pick(logits)
            else:
                logits = logits.float() / max(temperature, 1e-6)
                if top_k is not None:
                    kth = torch.topk(logits, top_k, dim=-1).values[:, -1:]
                    logits = logits.masked_fill(logits < kth, float("-inf"))
                if do_sample:
                    nxt = torch.multinomial(F.softmax(logits, dim=-1), 1)[:, 0]
                else:
                    nxt = logits.argmax(-1)
            if eos_token_id is not None:
                nxt = torch.where(finished, torch.full_like(nxt, eos_token_id), nxt)
                finished = finished | (nxt == eos_token_id)
            out.append(nxt.unsqueeze(1))
            if eos_token_id is not None and bool(finished.all()):
                break
            if dec.t >= dec.max_len:
                break
            logits = dec.step(nxt)
        return torch.cat(out, dim=1)

"""TEST INFRASTRUCTURE ONLY — the reference's eager PyTorch path, restated over a state dict.

A functional restatement (no nn.Module tree) of the reference model's eager forward and of its
eager incremental decoder, run on the CPU. It is the end-to-end checker for the HIP paths and the
timed CPU baseline of bench.py. Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline
leg import it. It uses the same torch operations as the reference's eager branch (roll, einsum,
scaled_dot_product_attention, rms_norm with eps=None, i.e. the fp32 epsilon), so its bf16 rounding points
are those of the reference.

Reference lines followed (/root/reference/dispatcher_hybrid/...):
  tree_mask               modeling_dispatcher.py:282-297, 311-323
  mixer                   modeling_dispatcher.py:63-123
  attention, rope         modeling_dispatcher.py:144-185
  swiglu, blocks          modeling_dispatcher.py:196-197, 210-212, 225-227
  forward                 modeling_dispatcher.py:325-351
  EagerDecoder.prefill    decoding.py:143-185 (tree), 225-245 (attention), 269-284
  EagerDecoder.step       decoding.py:187-222 (tree), 247-266 (attention), 286-304
"""

import math

import torch
import torch.nn.functional as F


class Spec:
    """Shape/behaviour fields of a DispatcherConfig (duck-typed: any object with these names)."""

    FIELDS = ("vocab_size", "d_model", "num_heads", "dim_feedforward", "num_layers", "max_len",
              "attn_layers", "attn_window", "doc_reset", "eot_token")

    def __init__(self, cfg):
        for f in self.FIELDS:
            setattr(self, f, getattr(cfg, f))
        self.attn_layers = tuple(self.attn_layers)
        self.levels = int(math.log2(self.max_len))
        self.head_dim = self.d_model // self.num_heads

    def is_attention(self, i):
        return self.attn_window > 0 and (i + 1) in self.attn_layers


def _norm(x, w):
    return F.rms_norm(x, (x.shape[-1],), w)                 # eps=None -> 2^-23 (fp32 math type)


def _w(sd, name):
    return sd[name]


def tree_mask(spec, ids, dtype):
    T = ids.shape[1]
    L = spec.levels
    mask = torch.zeros(T, L, dtype=dtype)
    for i in range(L):
        if 2 ** i < T:
            mask[2 ** i:, i] = 1.0
    if not spec.doc_reset:
        return mask
    is_eot = (ids == spec.eot_token).to(dtype)
    doc = torch.cumsum(is_eot, dim=1) - is_eot
    allowed = torch.stack([doc == torch.roll(doc, 2 ** i, dims=1) for i in range(L)], dim=-1).to(dtype)
    return mask.unsqueeze(0) * allowed


def n_levels(spec, T):
    return min(spec.levels, int(math.log2(T)) + 1)


def mixer(sd, pre, x, mask, spec, capture=None):
    """One mixer layer; `capture` (dict or None) receives A, B, V0 and the scanned V."""
    Bb, T, d = x.shape
    H, hd = spec.num_heads, spec.head_dim
    V0 = F.linear(x, _w(sd, pre + "linear_in.weight"))
    V = V0.view(Bb, T, H, hd).transpose(1, 2).reshape(Bb * H, T, hd)
    A = F.linear(x, _w(sd, pre + "gate_hidden.weight"))
    Bs = F.linear(x, _w(sd, pre + "gate_hidden_src.weight"))
    n_lv = n_levels(spec, T)
    if mask.dim() == 3:
        m4 = mask[..., :n_lv].unsqueeze(-1)
        mbh = mask[..., :n_lv].unsqueeze(1).expand(Bb, H, T, n_lv).reshape(Bb * H, T, n_lv)
    else:
        m4 = mask[:, :n_lv].view(1, T, n_lv, 1)
        mbh = mask[:, :n_lv]
    rolled = torch.stack([torch.roll(Bs, shifts=2 ** l, dims=1) for l in range(n_lv)], dim=2) * m4
    hidden = F.relu(A.unsqueeze(2) + rolled) ** 2
    pres = [torch.einsum("btld,lhd->btlh", hidden, _w(sd, pre + w)[:n_lv]) + _w(sd, pre + b)[:n_lv]
            for w, b in (("gate_out", "gate_out_bias"), ("forget_out", "forget_out_bias"),
                         ("reset_out", "reset_out_bias"))]

    def heads_first(p):
        return torch.sigmoid(p).permute(0, 3, 1, 2).reshape(Bb * H, T, n_lv).to(V.dtype)

    admit = heads_first(pres[0]) * mbh
    forget = heads_first(pres[1]) * mbh + (1.0 - mbh)
    transmit = heads_first(pres[2])
    for l in range(n_lv):
        if 2 ** l > T:
            break
        msg = torch.roll(transmit[..., l:l + 1] * V, shifts=2 ** l, dims=1)
        V = forget[..., l:l + 1] * V + admit[..., l:l + 1] * msg
    V = V.view(Bb, H, T, hd).transpose(1, 2).reshape(Bb, T, d)
    if capture is not None:
        capture.update(A=A, B=Bs, V0=V0, V=V, pre_i=pres[0], pre_f=pres[1], pre_r=pres[2])
    return F.linear(V, _w(sd, pre + "linear_out.weight"))


def rope_tables(spec, length, dtype):
    theta = 10000.0 ** (-torch.arange(0, spec.head_dim, 2, dtype=torch.float32) / spec.head_dim)
    ang = torch.arange(length, dtype=torch.float32)[:, None] * theta[None, :]
    return ang.cos().to(dtype), ang.sin().to(dtype)


def rope(x, cos, sin):
    x1, x2 = x[..., 0::2], x[..., 1::2]
    return torch.stack([x1 * cos - x2 * sin, x1 * sin + x2 * cos], dim=-1).flatten(-2)


def attention(sd, pre, x, spec):
    Bb, T, d = x.shape
    shape = (Bb, T, spec.num_heads, spec.head_dim)
    cos, sin = rope_tables(spec, T, x.dtype)
    q = rope(F.linear(x, _w(sd, pre + "linear_q.weight")).view(shape).transpose(1, 2), cos, sin)
    k = rope(F.linear(x, _w(sd, pre + "linear_k.weight")).view(shape).transpose(1, 2), cos, sin)
    v = F.linear(x, _w(sd, pre + "linear_v.weight")).view(shape).transpose(1, 2)
    if 0 < spec.attn_window < T:
        t = torch.arange(T)
        band = (t[:, None] >= t[None, :]) & (t[:, None] - t[None, :] < spec.attn_window)
        y = F.scaled_dot_product_attention(q, k, v, attn_mask=band)
    else:
        y = F.scaled_dot_product_attention(q, k, v, is_causal=True)
    return F.linear(y.transpose(1, 2).reshape(Bb, T, d), _w(sd, pre + "linear_out.weight"))


def swiglu(sd, pre, h):
    g = F.linear(h, _w(sd, pre + "linear_gate.weight"))
    u = F.linear(h, _w(sd, pre + "linear_up.weight"))
    return F.linear(F.silu(g) * u, _w(sd, pre + "linear_down.weight"))


def head_weight(sd):
    return sd["lm_head.weight"] if "lm_head.weight" in sd else sd["embedding.weight"]


@torch.no_grad()
def forward(sd, spec, ids, captures=None):
    """Logits (B, T, vocab) of the parallel eager forward. `captures`: optional dict that
    receives per-mixer-layer captures keyed by block index."""
    T = ids.shape[1]
    dtype = sd["embedding.weight"].dtype
    mask = tree_mask(spec, ids, dtype)
    x = F.embedding(ids, sd["embedding.weight"])
    for i in range(spec.num_layers):
        pre = f"blocks.{i}."
        h = _norm(x, sd[pre + "norm1.weight"])
        if spec.is_attention(i):
            x = x + attention(sd, pre + "attn.", h, spec)
        else:
            cap = {} if captures is not None else None
            x = x + mixer(sd, pre + "mixer.", h, mask, spec, cap)
            if captures is not None:
                captures[i] = cap
        x = x + swiglu(sd, pre + "ffn.", _norm(x, sd[pre + "norm2.weight"]))
    return F.linear(_norm(x, sd["norm_out.weight"]), head_weight(sd))


class EagerDecoder:
    """Exact eager incremental decoder over a state dict; caches use the reference layout
    (B_hist (B,Tmax,gh), rg_hist (B,Tmax,L,H), V_ring (B,S,d); K/V (B,Tmax,H,hd))."""

    def __init__(self, sd, spec, max_len=None):
        self.sd, self.spec = sd, spec
        self.max_len = max_len or spec.max_len
        self.dtype = sd["embedding.weight"].dtype
        self.t = 0

    def _slot(self, j, p):
        return (2 ** (j + 1) - 2) + (p & (2 ** (j + 1) - 1))

    def _alloc(self, Bb):
        sp, dt, Tm = self.spec, self.dtype, self.max_len
        L, H, hd, d = sp.levels, sp.num_heads, sp.head_dim, sp.d_model
        self.caches = []
        for i in range(sp.num_layers):
            if sp.is_attention(i):
                cos, sin = rope_tables(sp, Tm, dt)
                self.caches.append(dict(k=torch.zeros(Bb, Tm, H, hd, dtype=dt),
                                        v=torch.zeros(Bb, Tm, H, hd, dtype=dt), cos=cos, sin=sin))
            else:
                S = 2 ** (L + 1) - 2
                self.caches.append(dict(B_hist=torch.zeros(Bb, Tm, d, dtype=dt),
                                        rg_hist=torch.zeros(Bb, Tm, L, H, dtype=dt),
                                        V_ring=torch.zeros(Bb, S, d, dtype=dt), S=S))

    def _write_slab(self, c, j, slab):
        T = slab.shape[1]
        p0 = max(0, T - 2 ** (j + 1))
        pos = torch.arange(p0, T)
        c["V_ring"][:, self._slot(j, pos)] = slab[:, p0:]

    def _tree_prefill(self, pre, c, x):
        sd, sp = self.sd, self.spec
        Bb, T, d = x.shape
        L, H, hd = sp.levels, sp.num_heads, sp.head_dim
        m = pre + "mixer."
        h1 = _norm(x, sd[pre + "norm1.weight"])
        A = F.linear(h1, sd[m + "gate_hidden.weight"])
        Bs = F.linear(h1, sd[m + "gate_hidden_src.weight"])
        c["B_hist"][:, :T] = Bs
        n_lv = n_levels(sp, T) if T > 1 else 1
        V = F.linear(h1, sd[m + "linear_in.weight"]).view(Bb, T, H, hd)
        self._write_slab(c, 0, V.reshape(Bb, T, d))
        rolled = torch.stack([torch.roll(Bs, shifts=2 ** l, dims=1) for l in range(n_lv)], dim=2)
        wrap = torch.zeros(T, n_lv, 1, dtype=x.dtype)
        for l in range(n_lv):
            wrap[2 ** l:, l] = 1.0
        hidden = torch.relu(A.unsqueeze(2) + rolled * wrap) ** 2
        pi, pf, pr = (torch.einsum("btlg,lhg->btlh", hidden, sd[m + w][:n_lv]) + sd[m + b][:n_lv]
                      for w, b in (("gate_out", "gate_out_bias"), ("forget_out", "forget_out_bias"),
                                   ("reset_out", "reset_out_bias")))
        ig = torch.sigmoid(pi) * wrap
        fg = torch.sigmoid(pf) * wrap + (1.0 - wrap)
        rg = torch.sigmoid(pr)
        c["rg_hist"][:, :T, :n_lv] = rg
        if n_lv < L:
            hid0 = torch.relu(A) ** 2
            for l in range(n_lv, L):
                c["rg_hist"][:, :T, l] = torch.sigmoid(hid0 @ sd[m + "reset_out"][l].T + sd[m + "reset_out_bias"][l])
        for l in range(n_lv):
            msg = torch.roll(rg[:, :, l].unsqueeze(-1) * V, shifts=2 ** l, dims=1)
            V = fg[:, :, l].unsqueeze(-1) * V + ig[:, :, l].unsqueeze(-1) * msg
            if l + 1 < L:
                self._write_slab(c, l + 1, V.reshape(Bb, T, d))
        for j in range(n_lv + 1, L):
            self._write_slab(c, j, V.reshape(Bb, T, d))
        x = x + F.linear(V.reshape(Bb, T, d), sd[m + "linear_out.weight"])
        return x + swiglu(sd, pre + "ffn.", _norm(x, sd[pre + "norm2.weight"]))

    def _tree_step(self, pre, c, x, t):
        sd, sp = self.sd, self.spec
        Bb, d = x.shape
        L, H, hd = sp.levels, sp.num_heads, sp.head_dim
        m = pre + "mixer."
        h1 = _norm(x, sd[pre + "norm1.weight"])
        A = F.linear(h1, sd[m + "gate_hidden.weight"])
        c["B_hist"][:, t] = F.linear(h1, sd[m + "gate_hidden_src.weight"])
        V = F.linear(h1, sd[m + "linear_in.weight"]).view(Bb, H, hd)
        c["V_ring"][:, self._slot(0, t)] = V.reshape(Bb, -1)
        ar = torch.arange(L)
        src = t - torch.pow(2, ar)
        ok = src >= 0
        src_c = src.clamp(min=0)
        okf = ok.view(1, L, 1)
        hid = torch.relu(A.unsqueeze(1) + c["B_hist"][:, src_c] * okf) ** 2
        i_ = torch.sigmoid(torch.einsum("blg,lhg->blh", hid, sd[m + "gate_out"]) + sd[m + "gate_out_bias"]) * okf
        f_ = torch.sigmoid(torch.einsum("blg,lhg->blh", hid, sd[m + "forget_out"]) + sd[m + "forget_out_bias"])
        f_ = f_ * okf + (~okf).to(f_.dtype)
        r_ = torch.sigmoid(torch.einsum("blg,lhg->blh", hid, sd[m + "reset_out"]) + sd[m + "reset_out_bias"])
        c["rg_hist"][:, t] = r_
        rg_src = c["rg_hist"][:, src_c, ar]
        slots = (2 ** (ar + 1) - 2) + (src_c & (2 ** (ar + 1) - 1))
        msg = rg_src.unsqueeze(-1) * c["V_ring"][:, slots].view(Bb, L, H, hd)
        for l in range(L):
            V = f_[:, l].unsqueeze(-1) * V + i_[:, l].unsqueeze(-1) * msg[:, l]
            if l + 1 < L:
                c["V_ring"][:, self._slot(l + 1, t)] = V.reshape(Bb, -1)
        x = x + F.linear(V.reshape(Bb, -1), sd[m + "linear_out.weight"])
        return x + swiglu(sd, pre + "ffn.", _norm(x, sd[pre + "norm2.weight"]))

    def _attn_prefill(self, pre, c, x):
        sd, sp = self.sd, self.spec
        Bb, T, d = x.shape
        a = pre + "attn."
        h1 = _norm(x, sd[pre + "norm1.weight"])
        shape = (Bb, T, sp.num_heads, sp.head_dim)
        cos, sin = c["cos"][:T], c["sin"][:T]
        q = rope(F.linear(h1, sd[a + "linear_q.weight"]).view(shape).transpose(1, 2), cos, sin)
        k = rope(F.linear(h1, sd[a + "linear_k.weight"]).view(shape).transpose(1, 2), cos, sin)
        v = F.linear(h1, sd[a + "linear_v.weight"]).view(shape)
        c["k"][:, :T] = k.transpose(1, 2)
        c["v"][:, :T] = v
        vb = v.transpose(1, 2)
        if 0 < sp.attn_window < T:
            tt = torch.arange(T)
            band = (tt[:, None] >= tt[None, :]) & (tt[:, None] - tt[None, :] < sp.attn_window)
            y = F.scaled_dot_product_attention(q, k, vb, attn_mask=band)
        else:
            y = F.scaled_dot_product_attention(q, k, vb, is_causal=True)
        x = x + F.linear(y.transpose(1, 2).reshape(Bb, T, d), sd[a + "linear_out.weight"])
        return x + swiglu(sd, pre + "ffn.", _norm(x, sd[pre + "norm2.weight"]))

    def _attn_step(self, pre, c, x, t):
        sd, sp = self.sd, self.spec
        Bb = x.shape[0]
        a = pre + "attn."
        H, hd = sp.num_heads, sp.head_dim
        h1 = _norm(x, sd[pre + "norm1.weight"])
        cos, sin = c["cos"][t], c["sin"][t]
        q = rope(F.linear(h1, sd[a + "linear_q.weight"]).view(Bb, H, hd), cos, sin)
        c["k"][:, t] = rope(F.linear(h1, sd[a + "linear_k.weight"]).view(Bb, H, hd), cos, sin)
        c["v"][:, t] = F.linear(h1, sd[a + "linear_v.weight"]).view(Bb, H, hd)
        lo = max(0, t + 1 - sp.attn_window) if sp.attn_window > 0 else 0
        att = torch.softmax(torch.einsum("bhd,bthd->bht", q, c["k"][:, lo:t + 1]) / math.sqrt(hd), dim=-1)
        y = torch.einsum("bht,bthd->bhd", att, c["v"][:, lo:t + 1]).reshape(Bb, -1)
        x = x + F.linear(y, sd[a + "linear_out.weight"])
        return x + swiglu(sd, pre + "ffn.", _norm(x, sd[pre + "norm2.weight"]))

    @torch.no_grad()
    def prefill(self, ids):
        """ids (B, T) -> logits (B, T, vocab); fills the caches."""
        if bool((ids == self.spec.eot_token).any()) and self.spec.doc_reset:
            raise ValueError("prompt contains the document separator")
        Bb, T = ids.shape
        self._alloc(Bb)
        x = F.embedding(ids, self.sd["embedding.weight"])
        for i in range(self.spec.num_layers):
            pre = f"blocks.{i}."
            if self.spec.is_attention(i):
                x = self._attn_prefill(pre, self.caches[i], x)
            else:
                x = self._tree_prefill(pre, self.caches[i], x)
        self.t = T
        return F.linear(_norm(x, self.sd["norm_out.weight"]), head_weight(self.sd))

    @torch.no_grad()
    def step(self, tokens):
        """tokens (B,) -> logits (B, vocab) at position self.t."""
        if self.t >= self.max_len:
            raise ValueError("context exhausted")
        t = self.t
        x = F.embedding(tokens.view(-1), self.sd["embedding.weight"])
        for i in range(self.spec.num_layers):
            pre = f"blocks.{i}."
            if self.spec.is_attention(i):
                x = self._attn_step(pre, self.caches[i], x, t)
            else:
                x = self._tree_step(pre, self.caches[i], x, t)
        self.t = t + 1
        return F.linear(_norm(x, self.sd["norm_out.weight"]), head_weight(self.sd))

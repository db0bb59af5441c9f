"""TEST / BASELINE INFRASTRUCTURE ONLY -- never imported by the product path.

fp32 PyTorch-on-CPU restatement of the reference's chunked core
(src/prime_moment_attention/chunked_ssd.py:48-184) and of the step branch
(attention.py:119-143), used as the "PyTorch CPU path" timed beside the GPU in
bench.py and checked against the fp64 C oracle in tests/test_oracle.py.

Two inter-chunk carries are provided:
  carry="dense": the reference's lower-triangular (lambda^C)^(c-c'-1) matrix
                 applied to all chunk moments at once (chunked_ssd.py:113-126),
                 O(Nc^2) -- the reference's own cost;
  carry="scan":  the same recursion S^(c) = lambda^C S^(c-1) + dS^(c-1) as a
                 loop over chunks, O(Nc).
decay may be a float or one value per head (the reference takes one float).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def _per_head(lam, H):
    t = torch.as_tensor(lam, dtype=torch.float64).reshape(-1)
    return t.expand(H) if t.numel() == 1 else t


def chunked_core(q, k, v, lam, eps=1.0, chunk=64, state=None, carry="dense"):
    """q (pre-scaled by 1/sqrt(D)), k, v: fp32 [B, H, L, D] CPU tensors.
    Returns (y [B,H,L,D], state 6-tuple in the reference layout)."""
    B, H, L, D = q.shape
    C = chunk
    n = -(-L // C)
    pad = n * C - L
    lg = torch.log(_per_head(lam, H))                     # [H] fp64
    blk = lambda x: F.pad(x, (0, 0, 0, pad)).view(B, H, n, C, D)
    Q, K, V = blk(q), blk(k), blk(v)
    i = torch.arange(C, dtype=torch.float64)
    # intra-chunk lambda^(i-j) [i >= j] per head (chunked_ssd.py:79-87)
    gap = i[:, None] - i[None, :]
    mask = torch.where(gap >= 0, torch.exp(lg[:, None, None] * gap.clamp(min=0)), torch.zeros(()))
    mask = mask.float().view(1, H, 1, C, C)
    # Taylor block, numerator and row sums (chunked_ssd.py:89-94)
    Q2, K2 = Q * Q, K * K
    A = mask * (1.0 + Q @ K.transpose(-1, -2) + 0.5 * (Q2 @ K2.transpose(-1, -2)))
    num = A @ V
    den = A.sum(-1, keepdim=True)
    # chunk moment deltas with weights lambda^(C-1-j), zero on padding (:96-111)
    w = torch.exp(lg[:, None] * (C - 1 - i)[None, :]).float().view(1, H, 1, C, 1).expand(B, H, n, C, 1).clone()
    if pad:
        w[:, :, -1, C - pad:] = 0.0
    Kw, K2w = K * w, K2 * w
    dS0 = (V * w).sum(3)                                  # [B,H,n,D]
    dS1 = Kw.transpose(-1, -2) @ V                         # [B,H,n,D,D]
    dS2 = K2w.transpose(-1, -2) @ V
    dK0 = w.sum(3)                                         # [B,H,n,1]
    dK1, dK2 = Kw.sum(3), K2w.sum(3)
    deltas = (dS0, dS1, dS2, dK0, dK1, dK2)
    lamC = torch.exp(lg * C)                               # [H]
    if carry == "dense":
        c = torch.arange(n, dtype=torch.float64)
        e = c[:, None] - c[None, :] - 1
        Ad = torch.where(e >= 0, torch.exp(torch.log(lamC)[:, None, None] * e.clamp(min=0)), torch.zeros(()))
        Ad = Ad.float()                                    # [H, n, n]
        inter = [(Ad.view(1, H, n, n) @ d.reshape(B, H, n, -1)).view(d.shape) for d in deltas]
    else:
        inter = []
        for d in deltas:
            acc = torch.zeros_like(d[:, :, 0])
            out = torch.empty_like(d)
            lc = lamC.float().view(1, H, *([1] * (d.dim() - 3)))
            for ci in range(n):
                out[:, :, ci] = acc
                acc = lc * acc + d[:, :, ci]
            inter.append(out)
    if state is not None:                                  # incoming state (:128-137)
        c = torch.arange(n, dtype=torch.float64)
        for j, s in enumerate(state):
            s = s.reshape(inter[j][:, :, 0].shape)
            f = torch.exp(torch.log(lamC)[:, None] * c[None, :]).float()   # [H, n]
            inter[j] = inter[j] + s.unsqueeze(2) * f.view(1, H, n, *([1] * (s.dim() - 2)))
    iS0, iS1, iS2, iK0, iK1, iK2 = inter
    # readout of the carried state, scaled lambda^(i+1) (:139-157)
    into = torch.exp(lg[:, None] * (i + 1)[None, :]).float().view(1, H, 1, C, 1)
    Qi, Q2i = Q * into, Q2 * into
    cnum = iS0.unsqueeze(3) * into + Qi @ iS1 + 0.5 * (Q2i @ iS2)
    cden = (iK0.unsqueeze(3) * into + (Qi * iK1.unsqueeze(3)).sum(-1, keepdim=True)
            + 0.5 * (Q2i * iK2.unsqueeze(3)).sum(-1, keepdim=True))
    y = ((num + cnum) / (den + cden).clamp(min=eps)).reshape(B, H, n * C, D)[:, :, :L]
    # terminal state (:162-178): last carry decayed once more plus the last delta,
    # then the lambda^(-pad) correction for the zero-weighted padding
    corr = torch.exp(-lg * pad).float()
    fin = []
    for j in range(6):
        last = inter[j][:, :, -1] * lamC.float().view(1, H, *([1] * (inter[j].dim() - 3))) + deltas[j][:, :, -1]
        fin.append(last * corr.view(1, H, *([1] * (last.dim() - 2))))
    S0, S1, S2, K0, K1, K2 = fin
    return y, (S0, S1, S2, K0.reshape(B, H, 1), K1, K2)


def decode_step(q, k, v, lam, eps, state):
    """One step of attention.py:119-143 on CPU tensors ([B,H,D]); returns (y, state)."""
    B, H, D = q.shape
    lt = _per_head(lam, H).float().view(1, H, 1)
    S0, S1, S2, K0, K1, K2 = state
    k2 = k * k
    S0 = lt * S0 + v
    S1 = lt.unsqueeze(-1) * S1 + k.unsqueeze(-1) * v.unsqueeze(-2)
    S2 = lt.unsqueeze(-1) * S2 + k2.unsqueeze(-1) * v.unsqueeze(-2)
    K0 = lt * K0 + 1.0
    K1 = lt * K1 + k
    K2 = lt * K2 + k2
    q2 = q * q
    num = S0 + (q.unsqueeze(-2) @ S1).squeeze(-2) + 0.5 * (q2.unsqueeze(-2) @ S2).squeeze(-2)
    den = (K0 + (q * K1).sum(-1, keepdim=True) + 0.5 * (q2 * K2).sum(-1, keepdim=True)).clamp(min=eps)
    return num / den, (S0, S1, S2, K0, K1, K2)


class CausalLMCPU:
    """fp32 PyTorch-CPU restatement of the PRIME causal LM forward
    (model.py:47-68,101-120,163-200 of the reference) from a state dict in the
    reference's parameter names: RMSNorm -> q/k/v projections -> LayerNorm
    QK-norm -> q / sqrt(D) -> the chunked core above (the reference's O(Nc^2)
    carry) -> o_proj -> residual -> RMSNorm -> MLP (SwiGLU, or up/GELU/down
    when the state dict has no gate_proj) -> residual; final RMSNorm and the
    tied lm_head.  ``step`` is one token per sequence through the step formula
    (attention.py:119-143).  The timed CPU baseline of bench.py's model leg."""

    def __init__(self, state_dict, num_layers, num_heads, head_dim, decay, eps=1.0, rms_eps=1e-6, qk_norm=True,
                 round_bf16=False):
        self.W = {k: v.detach().to("cpu", torch.float32) for k, v in state_dict.items()}
        self.nl, self.H, self.D = num_layers, num_heads, head_dim
        self.decay, self.eps, self.rms_eps, self.qk_norm = decay, eps, rms_eps, qk_norm
        self.gelu = "layers.0.mlp.gate_proj.weight" not in self.W
        if "lm_head.weight" not in self.W:
            self.W["lm_head.weight"] = self.W["embed_tokens.weight"]
        # round_bf16: every activation a bf16 model stores (norm outputs,
        # projections, the QK-norm, the attention output, the GELU, the
        # residual stream after each add) is rounded to bf16 there, the
        # arithmetic in between staying fp32 -- the model in bf16 up to the
        # summation order of its products
        self.round_bf16 = round_bf16

    def _r(self, x):
        return x.to(torch.bfloat16).to(torch.float32) if self.round_bf16 else x

    def _rms(self, x, w):
        return self._r(x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + self.rms_eps) * w)

    def _mlp(self, p, x):
        W, r = self.W, self._r
        if self.gelu:
            return r(F.gelu(r(x @ W[p + "mlp.up_proj.weight"].T))) @ W[p + "mlp.down_proj.weight"].T
        return r(r(F.silu(r(x @ W[p + "mlp.gate_proj.weight"].T))) * r(x @ W[p + "mlp.up_proj.weight"].T)) \
            @ W[p + "mlp.down_proj.weight"].T

    def _qkv(self, p, h, B, L):
        W, H, D, r = self.W, self.H, self.D, self._r
        q = r(h @ W[p + "self_attn.q_proj.weight"].T).view(B, L, H, D).transpose(1, 2)
        k = r(h @ W[p + "self_attn.k_proj.weight"].T).view(B, L, H, D).transpose(1, 2)
        v = r(h @ W[p + "self_attn.v_proj.weight"].T).view(B, L, H, D).transpose(1, 2)
        if self.qk_norm:
            q = r(F.layer_norm(q, (D,), W[p + "self_attn.q_norm.weight"], W[p + "self_attn.q_norm.bias"]))
            k = r(F.layer_norm(k, (D,), W[p + "self_attn.k_norm.weight"], W[p + "self_attn.k_norm.bias"]))
        return r(q / D ** 0.5), k, v

    @torch.no_grad()
    def prefill(self, ids, carry="dense"):
        """ids [B, L] -> (last-position logits [B, V], per-layer states)."""
        W, r = self.W, self._r
        B, L = ids.shape
        x = W["embed_tokens.weight"][ids]
        states = []
        for i in range(self.nl):
            p = f"layers.{i}."
            q, k, v = self._qkv(p, self._rms(x, W[p + "input_layernorm.weight"]), B, L)
            y, st = chunked_core(q.contiguous(), k.contiguous(), v.contiguous(), self.decay, eps=self.eps,
                                 carry=carry)
            states.append(st)
            x = r(x + r(y).transpose(1, 2).reshape(B, L, -1) @ W[p + "self_attn.o_proj.weight"].T)
            x = r(x + self._mlp(p, self._rms(x, W[p + "post_attention_layernorm.weight"])))
        return r(self._rms(x[:, -1], W["norm.weight"]) @ W["lm_head.weight"].T), states

    @torch.no_grad()
    def step(self, tok, states):
        """tok [B] -> (logits [B, V], new states)."""
        W, r = self.W, self._r
        x = W["embed_tokens.weight"][tok]
        B = x.shape[0]
        new = []
        for i in range(self.nl):
            p = f"layers.{i}."
            q, k, v = self._qkv(p, self._rms(x, W[p + "input_layernorm.weight"])[:, None], B, 1)
            y, st = decode_step(q[:, :, 0], k[:, :, 0], v[:, :, 0], self.decay, self.eps, states[i])
            new.append(st)
            x = r(x + r(y).reshape(B, -1) @ W[p + "self_attn.o_proj.weight"].T)
            x = r(x + self._mlp(p, self._rms(x, W[p + "post_attention_layernorm.weight"])))
        return r(self._rms(x, W["norm.weight"]) @ W["lm_head.weight"].T), new

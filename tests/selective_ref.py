"""float64 torch composition of selective PRIME's recurrence, for torch
autograd to differentiate in the backward parity tests (not collected: no
test_ prefix).

It is the reference's parallel branch (selective.py:414-440: the [L, L]
decay matrix from the cumulative log decays, clamped at zero like
``(C_i - C_j).clamp(min=0)``, the beta-weighted moment similarities, the
row-sum denominator clamped at eps, and the end-of-call state from the decays
to the last token), extended by an incoming state in the selective convention
(S2 and K2 carry the 1/2): the state enters every token i with the decay
e^(c_i), c_i = sum_{t <= i} log lambda_t, exactly as the step branch
(selective.py:384-409) applies it one token at a time.  The CPU tests pin it
against the oracle's token-by-token restatement (oracle_selective_recurrent)."""
import torch


def selective_forward(q, k, v, log_decay, beta, eps, state=None):
    """q, k, v [B, H, L, D]; log_decay [B, H, L]; beta broadcastable to
    [B, H]; state: 6-tuple (S0 [B,H,D], S1, S2 [B,H,D,D], K0 [B,H,1],
    K1, K2 [B,H,D]) or None.  Returns (y [B,H,L,D], next_state)."""
    B, H, L, D = q.shape
    beta = beta.expand(B, H)
    b1 = beta[..., None, None]
    b2 = 0.5 * beta[..., None, None] ** 2
    c = torch.cumsum(log_decay, dim=-1)                                       # [B, H, L]
    mask = torch.tril(torch.ones(L, L, dtype=torch.bool))
    dm = torch.exp(-(c[..., None, :] - c[..., :, None]).clamp(min=0.0)) * mask  # [B, H, L, L]
    sim = 1.0 + b1 * (q @ k.transpose(-1, -2)) + b2 * ((q * q) @ (k * k).transpose(-1, -2))
    A = sim * dm
    num = A @ v
    den = A.sum(-1, keepdim=True)
    w_end = torch.exp(c[..., -1:] - c)[..., None]                             # [B, H, L, 1]
    ec = torch.exp(c)[..., None]                                              # [B, H, L, 1]
    S0 = (w_end * v).sum(2)
    S1 = b1 * ((k * w_end).transpose(-1, -2) @ v)
    S2 = b2 * (((k * k) * w_end).transpose(-1, -2) @ v)
    K0 = w_end.sum(2)
    K1 = beta[..., None] * (k * w_end).sum(2)
    K2 = 0.5 * beta[..., None] ** 2 * ((k * k) * w_end).sum(2)
    if state is not None:
        s0, s1, s2, k0, k1, k2 = state
        num = num + ec * (s0[:, :, None] + q @ s1 + (q * q) @ s2)
        den = den + ec * (k0[:, :, None] + (q * k1[:, :, None]).sum(-1, keepdim=True) +
                          ((q * q) * k2[:, :, None]).sum(-1, keepdim=True))
        e_end = torch.exp(c[..., -1])                                         # [B, H]
        S0 = S0 + e_end[..., None] * s0
        S1 = S1 + e_end[..., None, None] * s1
        S2 = S2 + e_end[..., None, None] * s2
        K0 = K0 + e_end[..., None] * k0
        K1 = K1 + e_end[..., None] * k1
        K2 = K2 + e_end[..., None] * k2
    y = num / den.clamp(min=eps)
    return y, (S0, S1, S2, K0, K1, K2)

"""TEST INFRASTRUCTURE: a torch restatement of the chunked gated delta-rule
PRIME forward (chunked_delta_prime.py:73-87 features, :177-283 chunk loop,
and the one-token step branch :140-176),
written as differentiable torch ops so that torch autograd (in fp64, on the
CPU) gives the reference gradients the HIP backward is checked against.  It is
pinned to the fp64 C oracle (oracle_delta_chunked, itself pinned by the
reference's own vectors in tests/golden/ref_delta.npz) by
tests/test_oracle.py::test_delta_torch_restatement_matches_oracle (the step:
test_delta_step_torch_restatement_matches_oracle, against oracle_delta_step),
and its autograd by central differences there.

q is pre-scaled (the module multiplies by 1/sqrt(D) before the features);
beta, alpha [B, H, L] per token and head; pad tokens of the last chunk carry
alpha = decay_pad and nothing else (chunked_delta_prime.py:181-188).
"""
import math

import torch
import torch.nn.functional as F


def features(q, k, eps=1e-5):
    """psi = [q, q^2/sqrt 2], phi = [k/|k|, (k^2/|k^2|)/sqrt 2] (chunked_delta_prime.py:73-87)."""
    kn = F.normalize(k, p=2, dim=-1, eps=eps)
    k2n = F.normalize(k * k, p=2, dim=-1, eps=eps)
    phi = torch.cat([kn, k2n / math.sqrt(2.0)], dim=-1)
    psi = torch.cat([q, q * q / math.sqrt(2.0)], dim=-1)
    return psi, phi


def delta_chunked(q, k, v, beta, alpha, decay_pad, eps=1e-5, bound=25.0, chunk=64, state=None):
    """y [B, H, L, D], final state [B, H, D, 2D] (chunked_delta_prime.py:177-283)."""
    B, H, L, D = q.shape
    psi, phi = features(q, k, eps)
    pad = (chunk - L % chunk) % chunk
    beta = beta.unsqueeze(-1)
    alpha = alpha.unsqueeze(-1)
    if pad:
        psi = F.pad(psi, (0, 0, 0, pad))
        phi = F.pad(phi, (0, 0, 0, pad))
        v = F.pad(v, (0, 0, 0, pad))
        beta = F.pad(beta, (0, 0, 0, pad))
        alpha = F.pad(alpha, (0, 0, 0, pad), value=decay_pad)
    n = (L + pad) // chunk
    C = chunk
    ch = lambda x: x.reshape(B, H, n, C, x.shape[-1])
    psi, phi, v, beta, alpha = ch(psi), ch(phi), ch(v), ch(beta), ch(alpha)
    cum = torch.cumsum(torch.log(torch.clamp(alpha, min=1e-5, max=1.0)), dim=3)
    cv = cum.squeeze(-1)
    tril = torch.tril(torch.ones(C, C, dtype=torch.bool))
    lam = torch.where(tril, torch.exp(cv.unsqueeze(-1) - cv.unsqueeze(-2)), torch.zeros((), dtype=q.dtype))
    gram = phi @ phi.transpose(-1, -2)
    strict = torch.tril(torch.ones(C, C, dtype=torch.bool), diagonal=-1)
    T = torch.where(strict, lam * gram * beta.transpose(-1, -2), torch.zeros((), dtype=q.dtype))
    T = T + torch.eye(C, dtype=q.dtype)
    S = torch.zeros(B, H, D, 2 * D, dtype=q.dtype) if state is None else state
    ys = []
    for c in range(n):
        into = torch.exp(cum[:, :, c])
        u = v[:, :, c] - (phi[:, :, c] * into) @ S.transpose(-1, -2)
        E = torch.linalg.solve_triangular(T[:, :, c], u, upper=False, unitriangular=True)
        att = torch.tril((psi[:, :, c] @ phi[:, :, c].transpose(-1, -2)) * lam[:, :, c])
        ys.append(att @ (beta[:, :, c] * E) + (psi[:, :, c] * into) @ S.transpose(-1, -2))
        end = cum[:, :, c, -1:, :]
        dS = (beta[:, :, c] * E).transpose(-1, -2) @ (phi[:, :, c] * torch.exp(end - cum[:, :, c]))
        S = S * torch.exp(end) + dS
        if bound > 0.0:
            nrm = torch.linalg.norm(S, dim=(-2, -1), keepdim=True)
            S = S * torch.clamp(bound / (nrm + 1e-6), max=1.0)
    y = torch.stack(ys, dim=2).reshape(B, H, n * C, D)[:, :, :L]
    return y, S


def delta_step(q, k, v, beta, alpha, eps=1e-5, bound=25.0, state=None):
    """The L == 1 branch (chunked_delta_prime.py:140-176): q, k, v [B, H, D]
    (q pre-scaled), beta, alpha [B, H]; predicts with the undecayed state,
    updates with alpha unclamped, clamps before the readout.  Returns
    y [B, H, D] and the new state [B, H, D, 2D]."""
    B, H, D = q.shape
    psi, phi = features(q, k, eps)
    S = torch.zeros(B, H, D, 2 * D, dtype=q.dtype) if state is None else state
    e = v - torch.einsum("bhde,bhe->bhd", S, phi)
    S = alpha[..., None, None] * S + torch.einsum("bhd,bhe->bhde", beta[..., None] * e, phi)
    if bound > 0.0:
        nrm = torch.linalg.norm(S, dim=(-2, -1), keepdim=True)
        S = S * torch.clamp(bound / (nrm + 1e-6), max=1.0)
    return torch.einsum("bhde,bhe->bhd", S, psi), S

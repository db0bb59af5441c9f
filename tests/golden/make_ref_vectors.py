"""Write golden input/output vectors from the reference PyTorch code.

Run ONLY in the build container, where /root/reference exists:
    python tests/golden/make_ref_vectors.py

It imports two reference files by path (attention.py with its chunked_ssd.py
dependency, and chunked_delta_prime.py) -- nothing else of the reference
package -- and writes small .npz fixtures next to this script.  Only behaviours
that no closed form or invariant pins are recorded here:

  ref_dense_state.npz  PrimeMomentAttention's dense branch (attention.py:160-202)
                       with an incoming state, where the denominator is clamped
                       before and after adding the carry (:177, :185);
  ref_delta.npz        ChunkedGatedDeltaPrimeAttention's chunked branch
                       (chunked_delta_prime.py:177-283) with the Lyapunov clamp
                       active (bound small enough to bite);
  ref_chunked_state.txt  whether chunked_prime_ssd_core accepts an incoming state
                       (it broadcasts 3-D state components against a 5-D decay
                       table, chunked_ssd.py:129-137).

The projections are set to block selections so the fixture holds core-level
tensors (q pre-scaled, k, v, state) rather than module weights.
"""
import importlib.util
import os
import sys

import numpy as np
import torch

REF = "/root/reference/src/prime_moment_attention"
OUT = os.path.dirname(os.path.abspath(__file__))


def _load(name, path):
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def _select(rows, cols, offset):
    w = torch.zeros(rows, cols)
    w[:, offset:offset + rows] = torch.eye(rows)
    return w


def dense_state():
    _load("chunked_ssd", os.path.join(REF, "chunked_ssd.py"))
    att = _load("ref_attention", os.path.join(REF, "attention.py"))
    H, D, L, B = 2, 16, 24, 2
    HD = H * D
    decay, eps = 0.97, 1.0
    m = att.PrimeMomentAttention(hidden_size=3 * HD, num_heads=H, head_dim=D, decay=decay,
                                 use_qk_norm=False, eps=eps)
    with torch.no_grad():
        m.q_proj.weight.copy_(_select(HD, 3 * HD, 0))
        m.k_proj.weight.copy_(_select(HD, 3 * HD, HD))
        m.v_proj.weight.copy_(_select(HD, 3 * HD, 2 * HD))
        m.o_proj.weight.copy_(_select(HD, 3 * HD, 0).T)
    g = torch.Generator().manual_seed(1234)
    # unnormalised q,k (|q.k/sqrt(D)| ~ 1) so that den < eps occurs for early tokens
    x = torch.randn(B, L, 3 * HD, generator=g)
    state = (torch.randn(B, H, D, generator=g), 0.05 * torch.randn(B, H, D, D, generator=g),
             0.05 * torch.randn(B, H, D, D, generator=g), 0.3 * torch.rand(B, H, 1, generator=g),
             0.05 * torch.randn(B, H, D, generator=g), 0.05 * torch.rand(B, H, D, generator=g))
    with torch.no_grad():
        out, nxt = m(x, state=state, return_state=True)
    q = x[..., :HD].view(B, L, H, D).transpose(1, 2) * m.scaling
    k = x[..., HD:2 * HD].view(B, L, H, D).transpose(1, 2)
    v = x[..., 2 * HD:].view(B, L, H, D).transpose(1, 2)
    y = out[..., :HD].view(B, L, H, D).transpose(1, 2)
    BH = B * H
    rec = dict(q=q.reshape(BH, L, D), k=k.reshape(BH, L, D), v=v.reshape(BH, L, D),
               y=y.reshape(BH, L, D), decay=np.float64(decay), eps=np.float64(eps))
    shapes = [(BH, D), (BH, D, D), (BH, D, D), (BH,), (BH, D), (BH, D)]
    for i in range(6):
        rec[f"s{i}"] = state[i].reshape(shapes[i])
        rec[f"o{i}"] = nxt[i].reshape(shapes[i])
    rec = {kk: (vv.double().numpy() if torch.is_tensor(vv) else vv) for kk, vv in rec.items()}
    np.savez_compressed(os.path.join(OUT, "ref_dense_state.npz"), **rec)

    # does the chunked core accept an incoming state?
    core = sys.modules["chunked_ssd"].chunked_prime_ssd_core
    msg = "accepted"
    try:
        core(q.float(), k.float(), v.float(), state=state, decay=decay, eps=eps, chunk_size=8,
             return_state=True)
    except Exception as e:  # record the reference behaviour, whatever it is
        msg = f"{type(e).__name__}: {e}"
    with open(os.path.join(OUT, "ref_chunked_state.txt"), "w") as f:
        f.write("chunked_prime_ssd_core(q,k,v,state=<6-tuple>, chunk_size=8) with "
                f"B={B},H={H},L={L},D={D}:\n{msg}\n")


def delta_clamp():
    dm = _load("ref_chunked_delta_prime", os.path.join(REF, "chunked_delta_prime.py"))
    H, D, L, B, C = 2, 16, 50, 1, 16
    HD = H * D
    decay, bound = 0.995, 2.0
    m = dm.ChunkedGatedDeltaPrimeAttention(hidden_size=5 * HD, num_heads=H, head_dim=D,
                                           chunk_size=C, decay=decay, use_qk_norm=False,
                                           lyapunov_bound=bound)
    with torch.no_grad():
        m.q_proj.weight.copy_(_select(HD, 5 * HD, 0))
        m.k_proj.weight.copy_(_select(HD, 5 * HD, HD))
        m.v_proj.weight.copy_(_select(HD, 5 * HD, 2 * HD))
        m.erase_proj.weight.copy_(_select(HD, 5 * HD, 3 * HD))
        m.write_proj.weight.copy_(_select(HD, 5 * HD, 4 * HD))
        m.o_proj.weight.copy_(_select(HD, 5 * HD, 0).T)
    g = torch.Generator().manual_seed(4321)
    x = torch.randn(B, L, 5 * HD, generator=g)
    x[..., 2 * HD:3 * HD] *= 4.0  # large values so that the clamp bites
    with torch.no_grad():
        out, S = m(x, return_state=True)
        q = x[..., :HD].view(B, L, H, D).transpose(1, 2) * m.scaling
        k = x[..., HD:2 * HD].view(B, L, H, D).transpose(1, 2)
        psi, phi = m._build_features(q.float(), k.float())
    v = x[..., 2 * HD:3 * HD].view(B, L, H, D).transpose(1, 2)
    be = torch.sigmoid(x[..., 3 * HD:4 * HD] - 2.5).view(B, L, H, D).transpose(1, 2)
    wr = torch.sigmoid(x[..., 4 * HD:] - 1.0).view(B, L, H, D).transpose(1, 2)
    beta = wr.mean(-1) * 0.5
    alpha = decay * (1.0 - be.mean(-1) * 0.5)
    y = out[..., :HD].view(B, L, H, D).transpose(1, 2)
    BH = B * H
    rec = dict(psi=psi.reshape(BH, L, 2 * D), phi=phi.reshape(BH, L, 2 * D),
               v=v.reshape(BH, L, D), beta=beta.reshape(BH, L), alpha=alpha.reshape(BH, L),
               y=y.reshape(BH, L, D), S=S.reshape(BH, D, 2 * D), q=q.reshape(BH, L, D),
               k=k.reshape(BH, L, D))
    rec = {kk: vv.double().numpy() for kk, vv in rec.items()}
    rec.update(decay=np.float64(decay), bound=np.float64(bound), chunk=np.int64(C))
    np.savez_compressed(os.path.join(OUT, "ref_delta.npz"), **rec)


if __name__ == "__main__":
    torch.manual_seed(0)
    dense_state()
    delta_clamp()
    print("wrote", sorted(f for f in os.listdir(OUT) if f.startswith("ref_")))

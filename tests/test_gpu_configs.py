"""GPU parity at the BASELINE workloads themselves (configs 1, 3, 4 and 5 at
their full shapes; config 2 is test_gpu_prefill.py::test_prefill_config2_shape_subset).

  config 1  fp32 B=1, H=12, L=512, lambda 0.9995: the HIP chunked core
            against the oracle recurrence (chunked_ssd.py:48-184 vs
            attention.py:119-143), fp32 tolerance
  config 3  decode B=512 x 12 layers x 12 heads, states pre-filled by the
            library's prefill of 1024 tokens: 64 random (layer, sequence,
            head) tiles against the oracle, every output finite
  config 4  the PRIME-125M-shaped LM at B=32 x 2048 (model.py:163-242)
  config 5  delta rule B=1, H=12, L=131072 (chunked_delta_prime.py:229-270):
            two heads in full against the oracle, all finite, |S|_F <= bound
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from prime_moment_attention import _lib

from gpu_util import TOL_BF16, TOL_F32, assert_close, assert_state_close, dev, state_to_np, to_dev, to_np

pytestmark = pytest.mark.gpu

D = 64
TOL_DECODE = 1e-4  # the decode arithmetic is fp32: one step against the oracle from the same state


def _qkv(shape, gen):
    """q, k, v ~ N(0,1) on the device; q and k L2-normalised over D, rounded to
    bf16, q / 8 (exact)."""
    out = []
    for i in range(3):
        x = torch.randn(*shape, generator=gen, device=dev())
        if i < 2:
            x = x / x.norm(dim=-1, keepdim=True).clamp_min(1e-12)
        x = x.to(torch.bfloat16)
        out.append(x / 8 if i == 0 else x)
    return out


# ------------------------------------------------------------------ config 1
def test_config1_fp32_chunked_core_matches_recurrence():
    """B=1, H=12, L=512, D=64, fp32 q/k/v ~ N(0,1) L2-normalised, lambda
    0.9995 for every head: the HIP chunked core (L=512 is not above the
    module's threshold, so the core is called directly) against the oracle
    recurrence, y and all six final states within 1e-3."""
    from prime_moment_attention import chunked_prime_ssd_core
    B, H, L = 1, 12, 512
    print(f"[config 1] B={B} H={H} L={L} fp32", flush=True)
    q, k, v = O.make_inputs((B, H, L, D), seed=1, bf16=False)
    y, st = chunked_prime_ssd_core(to_dev(q), to_dev(k), to_dev(v), decay=0.9995, eps=1.0, chunk_size=64,
                                   return_state=True)
    torch.cuda.synchronize()
    yo, so = O.recurrent(q.reshape(H, L, D), k.reshape(H, L, D), v.reshape(H, L, D), np.full(H, 0.9995), eps=1.0)
    assert y.dtype == torch.float32
    assert_close(to_np(y).reshape(H, L, D), yo, TOL_F32, "config 1 y")
    assert_state_close(state_to_np(st, H, D), so, TOL_F32, "config 1")


# ------------------------------------------------------------------ config 3
def test_config3_decode_b512_twelve_layers():
    """B=512 sequences x 12 layers x 12 heads; per-layer lambda_h ~
    U[0.99, 0.9999]; states pre-filled by the library's chunked prefill of
    1024 bf16 tokens; then 3 decode steps (one launch per layer, state in
    place).  64 random tiles: the prefilled state against the oracle
    recurrence (bf16 inputs), each decode step's y and state against one
    oracle step from the device state before it (fp32 arithmetic), and the
    final state against the oracle over all 1027 tokens; every y and state
    finite."""
    B, layers, H, P, steps = 512, 12, 12, 1024, 3
    print(f"[config 3] B={B} x {layers} layers x {H} heads, prefill {P}, {steps} steps", flush=True)
    gen = torch.Generator(device=dev()).manual_seed(3)
    rng = np.random.default_rng(3)
    lams = [rng.uniform(0.99, 0.9999, H).astype(np.float32) for _ in range(layers)]
    lam_d = [to_dev(x) for x in lams]
    tiles = sorted({(int(rng.integers(layers)), int(rng.integers(B)), int(rng.integers(H))) for _ in range(80)})[:64]
    assert len(tiles) == 64
    toks = {t: [] for t in tiles}  # per tile: the (q, k, v) rows it sees, float64
    states = [_lib.new_state(B, H, D, dev()) for _ in range(layers)]
    nb = 128
    for l in range(layers):
        for b0 in range(0, B, nb):
            q, k, v = _qkv((nb, H, P, D), gen)
            y = torch.empty_like(q)
            _lib.chunked_prefill(q, k, v, lam_d[l], 1.0, 64, None, y, tuple(s[b0:b0 + nb] for s in states[l]))
            for t in tiles:
                if t[0] == l and b0 <= t[1] < b0 + nb:
                    toks[t].append(tuple(to_np(x[t[1] - b0, t[2]]) for x in (q, k, v)))
            del q, k, v, y
    torch.cuda.synchronize()

    def tile_state(t):
        st = tuple(s[t[1], t[2]] for s in states[t[0]])
        return tuple(to_np(x)[None] for x in st)  # [1, ...] oracle layout (K0 [1, 1] -> reshaped below)

    def oracle_layout(st):
        return (st[0].reshape(1, D), st[1].reshape(1, D, D), st[2].reshape(1, D, D), st[3].reshape(1),
                st[4].reshape(1, D), st[5].reshape(1, D))

    # the prefilled states
    for t in tiles:
        q, k, v = (np.concatenate([x[i].reshape(-1, D) for x in toks[t]]).reshape(1, P, D) for i in range(3))
        _, so = O.recurrent(q, k, v, np.array([lams[t[0]][t[2]]], np.float64))
        assert_state_close(oracle_layout(tile_state(t)), so, TOL_BF16, f"prefilled tile {t}")
    for s in range(steps):
        before = {t: oracle_layout(tile_state(t)) for t in tiles}
        step_in = [_qkv((B, H, D), gen) for _ in range(layers)]
        ys = [torch.empty(B, H, D, device=dev()) for _ in range(layers)]  # fp32 y: the kernel's own precision
        for l in range(layers):
            _lib.decode_step(*step_in[l], lam_d[l], 1.0, states[l], states[l], ys[l])
        torch.cuda.synchronize()
        assert all(bool(torch.isfinite(y).all()) for y in ys), f"step {s}: non-finite y"
        for t in tiles:
            l, b, h = t
            qv, kv, vv = (to_np(x[b, h]).reshape(1, 1, D) for x in step_in[l])
            toks[t].append((qv[0, 0], kv[0, 0], vv[0, 0]))
            yo, so = O.recurrent(qv, kv, vv, np.array([lams[l][h]], np.float64), state=before[t])
            assert_close(to_np(ys[l][b, h]), yo[0, 0], TOL_DECODE, f"step {s} y {t}")
            assert_state_close(oracle_layout(tile_state(t)), so, TOL_DECODE, f"step {s} tile {t}")
    for st in states:
        assert all(bool(torch.isfinite(x).all()) for x in st)
    for t in tiles[:16]:
        q, k, v = (np.concatenate([x[i].reshape(-1, D) for x in toks[t]])[None] for i in range(3))
        assert q.shape == (1, P + steps, D)
        _, so = O.recurrent(q, k, v, np.array([lams[t[0]][t[2]]], np.float64))
        assert_state_close(oracle_layout(tile_state(t)), so, TOL_BF16, f"final tile {t}")


# ------------------------------------------------------------------ config 4
# The last token's logits of this random-init 12-layer bf16 model move by a
# few percent under any change of rounding: its residual stream is stored in
# bf16, so a sub-ulp change upstream flips whole ulps of single elements, and
# that grows through the layers (measured: swapping the library GEMMs of one
# step for correctly rounded ones moves its logits by 2.4%; a 2040-token
# prefill plus steps against one 2048-token prefill by 0.9-4.1% in relative
# L2).  The carried states, dominated by the 2040 prior tokens, agree to
# about 1e-3 and are held to the bf16 tolerance.
TOL_STEP_LOGITS = 1e-1
def test_config4_prime125m_full_shape():
    """PRIME-125M shape (12 layers, d_model 768, 12 x 64 heads, GELU MLP 3072,
    vocab 50304, bf16 weights, fp32 states), random init, B=32 x 2048 random
    ids (model.py:163-242).  The full prefill gives finite logits and states;
    the HIP-graph greedy decoder, the eager decoder and generate(temperature=0)
    give the same tokens over 8 steps (they run the same one-token step); on
    two sequences a prefill of 2040 tokens plus 8 recurrent steps continues
    one 2048-token prefill."""
    from prime_moment_attention import GreedyDecoder, PrimeForCausalLM, prime_125m_config
    cfg = prime_125m_config("gelu")
    torch.manual_seed(4)
    model = PrimeForCausalLM(cfg).to(device=dev(), dtype=torch.bfloat16).eval()
    gen = torch.Generator(device=dev()).manual_seed(4)
    B, L, n = 32, 2048, 8
    print(f"[config 4] PRIME-125M B={B} L={L}, {n} greedy steps", flush=True)
    ids = torch.randint(0, cfg.vocab_size, (B, L), device=dev(), generator=gen)
    with torch.no_grad():
        out = model(ids, return_states=True, logits_to_keep=1)
        torch.cuda.synchronize()
        assert torch.isfinite(out["logits"]).all()
        assert len(out["states"]) == 12
        assert all(bool(torch.isfinite(x).all()) for st in out["states"] for x in st)
        del out
    dg, de = GreedyDecoder(model, use_graph=True), GreedyDecoder(model, use_graph=False)
    tg, te = [dg.prefill(ids).clone()], [de.prefill(ids).clone()]
    for _ in range(n - 1):
        tg.append(dg.step().clone())
        te.append(de.step().clone())
    torch.cuda.synchronize()
    tg, te = torch.cat(tg, 1), torch.cat(te, 1)
    ref = model.generate(ids, max_new_tokens=n, temperature=0.0)[:, L:]
    assert torch.equal(tg, te)
    assert torch.equal(tg, ref), (tg != ref).sum()
    del dg, de
    # continuity: prefill + recurrent steps against one longer prefill
    with torch.no_grad():
        sub = ids[:2]
        full = model(sub, return_states=True)
        o = model(sub[:, :L - n], return_states=True, logits_to_keep=1)
        st = o["states"]
        for t in range(L - n, L):
            step = model(sub[:, t:t + 1], states=st, return_states=True)
            st = step["states"]
            a, r = step["logits"][:, -1].float(), full["logits"][:, t].float()
            l2 = float((a - r).norm() / r.norm())
            print(f"[config 4] step {t}: logits rel L2 {l2:.3e}", flush=True)
            assert l2 < TOL_STEP_LOGITS, (t, l2)
        for i in range(12):
            assert_state_close(state_to_np(st[i], 2 * 12, D), state_to_np(full["states"][i], 2 * 12, D), TOL_BF16,
                               f"layer {i} state after {n} steps")
    torch.cuda.synchronize()


# Parity of the whole model at the PRIME-125M shape against the fp32
# PyTorch-CPU restatement of the reference model (oracle/torch_cpu.py
# CausalLMCPU, model.py:47-200 with the chunked core of chunked_ssd.py:48-184
# and the step of attention.py:119-143), on the same weights and ids.  Two of
# the 32 sequences of the B=32 x 2048 prefill (the first and the last, so both
# halves of the paired split) and 8 teacher-forced decode steps (every side
# fed the GPU's greedy tokens) are recomputed on the CPU twice: in fp32, and
# with every activation the bf16 model stores rounded to bf16 where it stores
# it (the same model in bf16 up to the summation order of its products).
#   states: all 12 layers' final states within the bf16 input tolerance of
#     the fp32 restatement;
#   logits: the bf16 residual stream makes the last logits of this random-init
#     model move by percents under any change of rounding (single steps of one
#     sequence swing between 1e-2 and 1e-1 in relative L2 for every bf16 form
#     of the step, the bf16 emulation included), so the bound is the model's
#     own bf16 noise floor measured on the same inputs: the root mean square,
#     over the prefill and the 8 steps of both sequences, of the GPU's
#     relative L2 distance to the fp32 restatement may be at most
#     LOGITS_NOISE_FACTOR times that of the bf16 emulation; and no single
#     logits vector may be farther than LOGITS_MAX_REL_L2;
#   the greedy-token agreement with the fp32 restatement is printed.
LOGITS_NOISE_FACTOR = 2.0
LOGITS_MAX_REL_L2 = 0.25


def test_config4_prime125m_parity_against_fp32_restatement():
    from oracle.torch_cpu import CausalLMCPU
    from prime_moment_attention import PrimeForCausalLM, prime_125m_config
    cfg = prime_125m_config("gelu")
    torch.manual_seed(4)
    model = PrimeForCausalLM(cfg).to(device=dev(), dtype=torch.bfloat16).eval()
    gen = torch.Generator(device=dev()).manual_seed(4)
    B, L, pick, steps = 32, 2048, [0, 31], 8
    ids = torch.randint(0, cfg.vocab_size, (B, L), device=dev(), generator=gen)
    print(f"[config 4 parity] PRIME-125M B={B} L={L}, sequences {pick} and {steps} steps on the CPU", flush=True)
    with torch.no_grad():
        out = model(ids, return_states=True, logits_to_keep=1)
    torch.cuda.synchronize()
    logits = {"gpu": [out["logits"][pick, -1].float().cpu()]}
    gst = [tuple(t[pick].float().cpu() for t in st) for st in out["states"]]
    del out
    rel = lambda a, r: float((a - r).norm() / r.norm())
    # the GPU's decode steps on its greedy tokens (functional states)
    st_g = [tuple(t.to(dev()).contiguous() for t in s) for s in gst]
    toks = [logits["gpu"][0].argmax(-1)]
    for _ in range(steps):
        with torch.no_grad():
            o = model(toks[-1].view(-1, 1).to(dev()), states=st_g, return_states=True)
        st_g = o["states"]
        logits["gpu"].append(o["logits"][:, -1].float().cpu())
        toks.append(logits["gpu"][-1].argmax(-1))
    ids_c = ids[pick].cpu()
    for mode in ("fp32", "bf16"):
        cpu = CausalLMCPU(model.state_dict(), cfg.num_layers, cfg.num_heads, cfg.head_dim, cfg.decay, eps=cfg.eps,
                          rms_eps=cfg.rms_norm_eps, qk_norm=cfg.use_qk_norm, round_bf16=(mode == "bf16"))
        cl, cst = cpu.prefill(ids_c, carry="scan")
        if mode == "fp32":
            for i in range(cfg.num_layers):
                for c, (a, r) in enumerate(zip(gst[i], cst[i])):
                    e = float((a.reshape(r.shape) - r).abs().max() / r.abs().max().clamp_min(1e-30))
                    assert e < TOL_BF16, f"layer {i} state component {c}: rel err {e:.3e}"
        logits[mode] = [cl]
        for t in range(steps):
            cl, cst = cpu.step(toks[t], cst)
            logits[mode].append(cl)
    ref = logits["fp32"]
    agree = sum(int((g.argmax(-1) == r.argmax(-1)).sum()) for g, r in zip(logits["gpu"], ref))
    eg_all, eb_all = [], []
    for t in range(steps + 1):
        eg = [rel(logits["gpu"][t][i], ref[t][i]) for i in range(len(pick))]
        eb = [rel(logits["bf16"][t][i], ref[t][i]) for i in range(len(pick))]
        eg_all += eg
        eb_all += eb
        what = "prefill" if t == 0 else f"step {t}"
        print(f"[config 4 parity] {what}: logits rel L2 to the fp32 restatement per sequence: GPU "
              f"{' '.join(f'{e:.2e}' for e in eg)}, bf16 emulation {' '.join(f'{e:.2e}' for e in eb)}", flush=True)
    rms = lambda v: (sum(e * e for e in v) / len(v)) ** 0.5
    print(f"[config 4 parity] rms rel L2: GPU {rms(eg_all):.3e}, bf16 emulation {rms(eb_all):.3e}; greedy "
          f"agreement with the fp32 restatement {agree}/{(steps + 1) * len(pick)}", flush=True)
    assert rms(eg_all) <= LOGITS_NOISE_FACTOR * rms(eb_all), (rms(eg_all), rms(eb_all))
    assert max(eg_all) <= LOGITS_MAX_REL_L2, max(eg_all)


# ------------------------------------------------------------------ config 5
def test_config5_delta_long_context():
    """B=1, H=12, D=64, L=131072, chunk 64: bf16 q/k/v (N(0,1), QK-normed,
    q / 8), beta ~ sigmoid(N(0,1)) per token and head, alpha = per-head lambda
    ~ U[0.99, 0.9999], Lyapunov bound 25.  Heads 0 and 11 in full against the
    oracle (y and the final state); every head's y finite and its final state
    within the bound."""
    B, H, L, bound = 1, 12, 131072, 25.0
    print(f"[config 5] delta B={B} H={H} L={L}", flush=True)
    q, k, v = O.make_inputs((B, H, L, D), seed=5, bf16=True)
    rng = np.random.default_rng(5)
    beta = (1.0 / (1.0 + np.exp(-rng.standard_normal((B, H, L))))).astype(np.float32)
    lam = rng.uniform(0.99, 0.9999, H).astype(np.float32)
    alpha = np.ascontiguousarray(np.broadcast_to(lam[None, :, None], (B, H, L))).astype(np.float32)
    y = torch.empty(B, H, L, D, device=dev(), dtype=torch.bfloat16)
    s = torch.empty(B, H, D, 2 * D, device=dev())
    _lib.delta_prefill(to_dev(q, torch.bfloat16), to_dev(k, torch.bfloat16), to_dev(v, torch.bfloat16),
                       to_dev(beta), to_dev(alpha), 0.9995, 1e-5, bound, None, y, s)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(y).all()) and bool(torch.isfinite(s).all())
    norms = s.norm(dim=(2, 3)).flatten()
    assert float(norms.max()) <= bound * (1 + 1e-5), norms
    yn, sn = to_np(y)[0], to_np(s)[0]
    for h in (0, 11):
        psi, phi = O.delta_features(q[0, h][None], k[0, h][None], eps=1e-5)
        yo, so = O.delta_chunked(psi, phi, v[0, h][None], beta[0, h][None], alpha[0, h][None], 0.9995, bound=bound,
                                 chunk=64)
        assert_close(yn[h], yo[0], TOL_BF16, f"config 5 y head {h}")
        assert_close(sn[h], so[0], TOL_BF16, f"config 5 S head {h}")

"""ctypes binding of libprime_mi355x.so (the C ABI in include/prime_mi355x.h).

This is the only route from Python to the compute: there is no CPU or eager
fallback.  If the library is missing, or a tensor is not on a HIP device, the
calls raise.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional, Sequence, Tuple

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libprime_mi355x.so")

PRIME_F32, PRIME_BF16, PRIME_F16 = 0, 1, 2
PRIME_FLAG_DENSE_CLAMP = 1
ABI_VERSION = 1

_DTYPES = {torch.float32: PRIME_F32, torch.bfloat16: PRIME_BF16, torch.float16: PRIME_F16}

# every symbol include/prime_mi355x.h declares
EXPORTS = ("prime_abi_version", "prime_last_error", "prime_decode_step", "prime_chunked_prefill",
           "prime_chunked_prefill_workspace_size", "prime_timer_enable", "prime_timer_reset",
           "prime_timer_read", "prime_delta_prefill", "prime_delta_prefill_workspace_size",
           "prime_delta_decode_step", "prime_decode_step_qknorm", "prime_add_rmsnorm", "prime_gelu", "prime_selective_log_decay", "prime_argmax",
           "prime_head_layernorm", "prime_linear", "prime_linear_residual", "prime_linear_fused", "prime_selective_prefill",
           "prime_selective_decode_step", "prime_accumulate", "prime_accumulate_workspace_size",
           "prime_decode_readout", "prime_decode_update", "prime_chunked_prefill_backward",
           "prime_chunked_prefill_backward_workspace_size", "prime_chunked_prefill_qknorm",
           "prime_selective_prefill_qknorm", "prime_accumulate_noalloc", "prime_selective_prefill_backward",
           "prime_selective_prefill_backward_workspace_size", "prime_hbm_stream",
           "prime_frag_rows", "prime_pack_frag", "prime_linear_frag_workspace_size", "prime_linear_frag",
           "prime_delta_prefill_backward", "prime_delta_prefill_backward_workspace_size",
           "prime_delta_decode_step_backward")

# bytes of the fixed device scratch behind prime_accumulate_noalloc
NOALLOC_SCRATCH_BYTES = 32 << 20

# kernel identifiers of the launch timer
KERNEL_PREFILL_CHUNKS, KERNEL_PREFILL_SEGMENTS, KERNEL_SEGMENT_SCAN, KERNEL_DECODE = 0, 1, 2, 3
KERNEL_DELTA_PREP, KERNEL_DELTA_SCAN, KERNEL_DELTA_STEP = 4, 5, 6
KERNEL_BWD_DQ, KERNEL_BWD_DKV, KERNEL_BWD_DUAL, KERNEL_BWD_DUAL_SCAN = 7, 8, 9, 10
KERNEL_NAMES = {KERNEL_PREFILL_CHUNKS: "prefill_bf16_kernel (fused chunk loop)", KERNEL_PREFILL_SEGMENTS:
                "prefill_bf16_kernel (segment states)", KERNEL_SEGMENT_SCAN: "segment_scan_kernel",
                KERNEL_DECODE: "decode_step_kernel", KERNEL_DELTA_PREP: "delta_prep_kernel",
                KERNEL_DELTA_SCAN: "delta_scan_kernel", KERNEL_DELTA_STEP: "delta_step_kernel",
                KERNEL_BWD_DQ: "prefill_bwd_dq_kernel", KERNEL_BWD_DKV: "prefill_bwd_dkv_kernel<false>",
                KERNEL_BWD_DUAL: "prefill_bwd_dkv_kernel<true>", KERNEL_BWD_DUAL_SCAN: "bwd_dual_scan_kernel"}


class PrimeTensor(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("dtype", ctypes.c_int32), ("layout", ctypes.c_int32),
                ("stride_b", ctypes.c_int64), ("stride_h", ctypes.c_int64), ("stride_l", ctypes.c_int64)]


class PrimeState(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in ("s0", "s1", "s2", "k0", "k1", "k2")]


class PrimeQkNorm(ctypes.Structure):
    _fields_ = [("q_weight", ctypes.c_void_p), ("q_bias", ctypes.c_void_p), ("k_weight", ctypes.c_void_p),
                ("k_bias", ctypes.c_void_p), ("dtype", ctypes.c_int32), ("eps", ctypes.c_float),
                ("q_scale", ctypes.c_float)]


class PrimeSelectiveGate(ctypes.Structure):
    _fields_ = [("decay", ctypes.c_void_p), ("step", ctypes.c_void_p), ("step_dtype", ctypes.c_int32),
                ("reserved", ctypes.c_int32), ("step_sb", ctypes.c_int64), ("tau", ctypes.c_void_p),
                ("step_min", ctypes.c_float), ("step_max", ctypes.c_float)]


_lib = None


def load() -> ctypes.CDLL:
    """Load the HIP library (no GPU needed to load it)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"PRIME HIP library not built: {LIB_PATH} is missing "
                           "(run __graft_entry__.build() or make -C prime-moment-attention_amd)")
    L = ctypes.CDLL(LIB_PATH)
    L.prime_abi_version.restype = ctypes.c_int
    L.prime_last_error.restype = ctypes.c_char_p
    P = ctypes.POINTER
    L.prime_decode_step.argtypes = [P(PrimeTensor)] * 3 + [ctypes.c_int] * 4 + [
        ctypes.c_void_p, ctypes.c_float, P(PrimeState), P(PrimeState), P(PrimeTensor), ctypes.c_void_p]
    L.prime_decode_step.restype = ctypes.c_int
    L.prime_chunked_prefill.argtypes = [P(PrimeTensor)] * 3 + [ctypes.c_int] * 6 + [
        ctypes.c_void_p, ctypes.c_float, ctypes.c_uint, P(PrimeState), P(PrimeTensor),
        P(PrimeState), ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
    L.prime_chunked_prefill.restype = ctypes.c_int
    L.prime_chunked_prefill_workspace_size.argtypes = [ctypes.c_int] * 3 + [ctypes.c_uint]
    L.prime_chunked_prefill_workspace_size.restype = ctypes.c_size_t
    L.prime_timer_enable.argtypes = [ctypes.c_uint]
    fp = ctypes.c_void_p
    L.prime_delta_prefill.argtypes = [P(PrimeTensor)] * 3 + [fp, fp] + [ctypes.c_int] * 6 + [
        ctypes.c_float] * 3 + [fp, P(PrimeTensor), fp, fp, ctypes.c_size_t, fp]
    L.prime_delta_prefill.restype = ctypes.c_int
    L.prime_delta_prefill_workspace_size.argtypes = [ctypes.c_int] * 3 + [ctypes.c_uint]
    L.prime_delta_prefill_workspace_size.restype = ctypes.c_size_t
    L.prime_delta_decode_step.argtypes = [P(PrimeTensor)] * 3 + [fp, fp] + [ctypes.c_int] * 4 + [
        ctypes.c_float] * 2 + [fp, fp, P(PrimeTensor), fp]
    L.prime_delta_decode_step.restype = ctypes.c_int
    L.prime_delta_decode_step_backward.argtypes = [P(PrimeTensor)] * 3 + [fp, fp] + [ctypes.c_int] * 4 + [
        ctypes.c_float] * 2 + [fp, P(PrimeTensor)] + [fp] * 7 + [fp]
    L.prime_delta_decode_step_backward.restype = ctypes.c_int
    L.prime_decode_step_qknorm.argtypes = [P(PrimeTensor)] * 3 + [ctypes.c_int] * 4 + [
        ctypes.c_void_p, ctypes.c_float, P(PrimeQkNorm), P(PrimeState), P(PrimeState), P(PrimeTensor), ctypes.c_void_p]
    L.prime_decode_step_qknorm.restype = ctypes.c_int
    L.prime_add_rmsnorm.argtypes = [fp] * 4 + [ctypes.c_int] * 3 + [ctypes.c_float, fp]
    L.prime_add_rmsnorm.restype = ctypes.c_int
    L.prime_gelu.argtypes = [fp, fp, ctypes.c_int64, ctypes.c_int, fp]
    L.prime_gelu.restype = ctypes.c_int
    L.prime_selective_log_decay.argtypes = [fp, ctypes.c_int, ctypes.c_int64, ctypes.c_int64, fp, ctypes.c_float,
                                            ctypes.c_float, ctypes.c_int, ctypes.c_int, ctypes.c_int, fp, fp]
    L.prime_selective_log_decay.restype = ctypes.c_int
    L.prime_argmax.argtypes = [fp, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int64, fp, fp]
    L.prime_argmax.restype = ctypes.c_int
    L.prime_head_layernorm.argtypes = [P(PrimeTensor)] * 2 + [ctypes.c_int] * 4 + [fp, fp, ctypes.c_int,
                                                                                 ctypes.c_float, ctypes.c_float, fp]
    L.prime_head_layernorm.restype = ctypes.c_int
    L.prime_linear.argtypes = [fp, fp, fp] + [ctypes.c_int] * 3 + [ctypes.c_int64] * 3 + [ctypes.c_int] * 2 + [fp]
    L.prime_linear.restype = ctypes.c_int
    L.prime_linear_residual.argtypes = [fp] * 4 + [ctypes.c_int] * 3 + [ctypes.c_int64] * 4 + [ctypes.c_int, fp]
    L.prime_linear_residual.restype = ctypes.c_int
    L.prime_linear_fused.argtypes = [fp] * 4 + [ctypes.c_int] * 3 + [ctypes.c_int64] * 4 + [ctypes.c_int] * 2 + [
        ctypes.c_float, fp]
    L.prime_linear_fused.restype = ctypes.c_int
    L.prime_selective_prefill.argtypes = [P(PrimeTensor)] * 3 + [ctypes.c_int] * 5 + [
        ctypes.c_void_p, ctypes.c_void_p, ctypes.c_float, P(PrimeState), P(PrimeTensor), P(PrimeState),
        ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
    L.prime_selective_prefill.restype = ctypes.c_int
    L.prime_chunked_prefill_qknorm.argtypes = [P(PrimeTensor)] * 3 + [ctypes.c_int] * 6 + [
        ctypes.c_void_p, ctypes.c_float, ctypes.c_uint, P(PrimeQkNorm), P(PrimeState), P(PrimeTensor),
        P(PrimeState), ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
    L.prime_chunked_prefill_qknorm.restype = ctypes.c_int
    L.prime_selective_prefill_qknorm.argtypes = [P(PrimeTensor)] * 3 + [ctypes.c_int] * 5 + [
        ctypes.c_void_p, ctypes.c_void_p, ctypes.c_float, P(PrimeQkNorm), P(PrimeState), P(PrimeTensor),
        P(PrimeState), ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
    L.prime_selective_prefill_qknorm.restype = ctypes.c_int
    L.prime_selective_decode_step.argtypes = [P(PrimeTensor)] * 3 + [ctypes.c_int] * 4 + [
        P(PrimeSelectiveGate), ctypes.c_void_p, ctypes.c_float, P(PrimeQkNorm), P(PrimeState), P(PrimeState),
        P(PrimeTensor), ctypes.c_void_p]
    L.prime_selective_decode_step.restype = ctypes.c_int
    L.prime_accumulate.argtypes = [P(PrimeTensor)] * 2 + [ctypes.c_int] * 5 + [
        fp, P(PrimeState), P(PrimeState), fp, ctypes.c_size_t, fp]
    L.prime_accumulate.restype = ctypes.c_int
    L.prime_accumulate_noalloc.argtypes = [P(PrimeTensor)] * 2 + [ctypes.c_int] * 5 + [
        fp, P(PrimeState), P(PrimeState), fp]
    L.prime_accumulate_noalloc.restype = ctypes.c_int
    L.prime_accumulate_workspace_size.argtypes = [ctypes.c_int] * 3
    L.prime_accumulate_workspace_size.restype = ctypes.c_size_t
    L.prime_decode_readout.argtypes = [P(PrimeTensor)] + [ctypes.c_int] * 3 + [
        ctypes.c_float, P(PrimeState), P(PrimeTensor), fp]
    L.prime_decode_readout.restype = ctypes.c_int
    L.prime_decode_update.argtypes = [P(PrimeTensor)] * 2 + [ctypes.c_int] * 4 + [
        fp, P(PrimeState), P(PrimeState), fp]
    L.prime_decode_update.restype = ctypes.c_int
    L.prime_chunked_prefill_backward.argtypes = [P(PrimeTensor)] * 3 + [ctypes.c_int] * 5 + [
        fp, ctypes.c_float, ctypes.c_uint, P(PrimeState), P(PrimeTensor), P(PrimeState)] + [
        P(PrimeTensor)] * 3 + [P(PrimeState), fp, ctypes.c_size_t, fp]
    L.prime_chunked_prefill_backward.restype = ctypes.c_int
    L.prime_chunked_prefill_backward_workspace_size.argtypes = [ctypes.c_int] * 3
    L.prime_chunked_prefill_backward_workspace_size.restype = ctypes.c_size_t
    L.prime_selective_prefill_backward.argtypes = [P(PrimeTensor)] * 3 + [ctypes.c_int] * 5 + [
        fp, fp, ctypes.c_float, P(PrimeState), P(PrimeTensor), P(PrimeState)] + [P(PrimeTensor)] * 3 + [
        P(PrimeState), fp, fp, fp, ctypes.c_size_t, fp]
    L.prime_selective_prefill_backward.restype = ctypes.c_int
    L.prime_selective_prefill_backward_workspace_size.argtypes = [ctypes.c_int] * 3
    L.prime_selective_prefill_backward_workspace_size.restype = ctypes.c_size_t
    L.prime_timer_read.argtypes = [ctypes.c_int, P(ctypes.c_double), P(ctypes.c_int64)]
    L.prime_hbm_stream.argtypes = [fp, fp, ctypes.c_size_t, ctypes.c_int, ctypes.c_int, fp]
    L.prime_hbm_stream.restype = ctypes.c_int
    L.prime_delta_prefill_backward_workspace_size.argtypes = [ctypes.c_int] * 5
    L.prime_delta_prefill_backward_workspace_size.restype = ctypes.c_size_t
    L.prime_delta_prefill_backward.argtypes = [P(PrimeTensor)] * 3 + [fp, fp] + [ctypes.c_int] * 6 + [
        ctypes.c_float] * 3 + [fp, P(PrimeTensor)] + [fp] * 8 + [ctypes.c_size_t, fp]
    L.prime_delta_prefill_backward.restype = ctypes.c_int
    L.prime_frag_rows.argtypes = [ctypes.c_int]
    L.prime_frag_rows.restype = ctypes.c_int
    L.prime_pack_frag.argtypes = [fp, ctypes.c_int64, ctypes.c_int64, fp, ctypes.c_int, ctypes.c_int, fp, fp]
    L.prime_pack_frag.restype = ctypes.c_int
    L.prime_linear_frag_workspace_size.argtypes = [ctypes.c_int] * 3
    L.prime_linear_frag_workspace_size.restype = ctypes.c_size_t
    L.prime_linear_frag.argtypes = [fp] * 4 + [ctypes.c_int] * 3 + [ctypes.c_int64, ctypes.c_int, ctypes.c_uint,
                                                                   ctypes.c_float, fp, fp, fp, ctypes.c_size_t, fp]
    L.prime_linear_frag.restype = ctypes.c_int
    v = L.prime_abi_version()
    if v != ABI_VERSION:
        raise RuntimeError(f"libprime_mi355x ABI {v} != expected {ABI_VERSION}")
    _lib = L
    return L


def last_error() -> str:
    return load().prime_last_error().decode(errors="replace")


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what} failed ({rc}): {last_error()}")


def _dev_check(*ts: torch.Tensor) -> None:
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError("PRIME kernels need tensors on a HIP device (no CPU fallback)")


def _shape(t: torch.Tensor, shape, name: str) -> None:
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} has shape {tuple(t.shape)}, expected {tuple(shape)}")


def _check_decay(decay: torch.Tensor, H: int) -> None:
    if decay.dtype != torch.float32 or decay.numel() != H or not decay.is_contiguous():
        raise ValueError(f"decay must be a contiguous fp32 tensor of {H} values")


def _check_state(state, B: int, H: int, D: int, name: str) -> None:
    if state is None:
        return
    shapes = [(B, H, D), (B, H, D, D), (B, H, D, D), (B, H, 1), (B, H, D), (B, H, D)]
    if len(state) != 6:
        raise ValueError(f"{name} must be a 6-tuple")
    for t, sh in zip(state, shapes):
        if t.dtype != torch.float32 or not t.is_contiguous() or t.numel() != B * H * _prod(sh[2:]):
            raise ValueError(f"{name}: component of shape {tuple(t.shape)} / {t.dtype} is not a "
                             f"contiguous fp32 {sh}")
        _dev_check(t)


PRIME_LAYOUT_STRIDED, PRIME_LAYOUT_FRAG = 0, 1


def frag_desc(y: torch.Tensor) -> PrimeTensor:
    """Descriptor of a decode-step output held in the fragment layout (a flat
    bf16 buffer of frag_rows(B) x H*D elements)."""
    if y.dtype != torch.bfloat16 or not y.is_contiguous():
        raise ValueError("a fragment-layout y is a contiguous bf16 buffer")
    return PrimeTensor(y.data_ptr(), PRIME_BF16, PRIME_LAYOUT_FRAG, 0, 0, 0)


def _y_desc(y, B, H, D, y_frag):
    if not y_frag:
        _shape(y, (B, H, D), "y")
        return tensor_desc(y, False)
    if y.numel() < frag_rows(B) * H * D:
        raise ValueError(f"fragment-layout y needs {frag_rows(B) * H * D} elements")
    return frag_desc(y)


def tensor_desc(x: torch.Tensor, has_l: bool) -> PrimeTensor:
    """Descriptor of a [B, H, L, D] (has_l) or [B, H, D] view; D must be contiguous."""
    if x.dtype not in _DTYPES:
        raise RuntimeError(f"unsupported dtype {x.dtype}")
    if x.stride(-1) != 1:
        raise RuntimeError("innermost (head) dimension must be contiguous")
    sb, sh = x.stride(0), x.stride(1)
    sl = x.stride(2) if has_l else 0
    return PrimeTensor(x.data_ptr(), _DTYPES[x.dtype], 0, sb, sh, sl)


def state_desc(state: Optional[Sequence[torch.Tensor]]) -> Optional[PrimeState]:
    if state is None:
        return None
    return PrimeState(*[t.data_ptr() for t in state])


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def bind_decode_step(q, k, v, decay: torch.Tensor, eps: float, state_in, state_out, y):
    """Validate once and return a no-argument callable that launches
    prime_decode_step on these exact buffers (on the device's current stream
    at call time).  For tight loops whose buffers are fixed (generation, benchmarks):
    the call skips the Python-side checks and descriptor building."""
    _decode_checks(q, k, v, decay, state_in, state_out, y)
    L = load()
    B, H, D = q.shape
    refs = (tensor_desc(q, False), tensor_desc(k, False), tensor_desc(v, False), state_desc(state_in),
            state_desc(state_out), tensor_desc(y, False))
    args = (ctypes.byref(refs[0]), ctypes.byref(refs[1]), ctypes.byref(refs[2]), B, H, k.shape[1], D,
            ctypes.c_void_p(decay.data_ptr()), ctypes.c_float(eps),
            ctypes.byref(refs[3]) if refs[3] else None, ctypes.byref(refs[4]), ctypes.byref(refs[5]))
    fn, dev = L.prime_decode_step, q.device
    keep = (q, k, v, decay, state_in, state_out, y, refs)

    def launch():
        _check(fn(*args, torch.cuda.current_stream(dev).cuda_stream), "prime_decode_step")
    launch.buffers = keep
    return launch


def _decode_checks(q, k, v, decay, state_in, state_out, y, y_frag=False):
    _dev_check(q, k, v, y, decay)
    B, H, D = q.shape
    Hkv = k.shape[1]
    _shape(k, (B, Hkv, D), "k")
    _shape(v, (B, Hkv, D), "v")
    if not y_frag:
        _shape(y, (B, H, D), "y")
    _check_decay(decay, H)
    _check_state(state_in, B, H, D, "state_in")
    _check_state(state_out, B, H, D, "state_out")


def decode_step(q, k, v, decay: torch.Tensor, eps: float, state_in, state_out, y) -> None:
    """One fused decode step (prime_decode_step).  q [B,H,D], k/v [B,Hkv,D],
    decay fp32 [H] on device, states: 6-tuples of contiguous fp32 tensors."""
    _decode_checks(q, k, v, decay, state_in, state_out, y)
    B, H, D = q.shape
    L = load()
    qd, kd, vd, yd = tensor_desc(q, False), tensor_desc(k, False), tensor_desc(v, False), tensor_desc(y, False)
    si, so = state_desc(state_in), state_desc(state_out)
    rc = L.prime_decode_step(ctypes.byref(qd), ctypes.byref(kd), ctypes.byref(vd), B, H, k.shape[1], D,
                             decay.data_ptr(), float(eps), ctypes.byref(si) if si else None,
                             ctypes.byref(so), ctypes.byref(yd), _stream(q.device))
    _check(rc, "prime_decode_step")


def qk_norm(q_norm, k_norm, q_scale: float, dtype) -> PrimeQkNorm:
    """prime_qk_norm_t for two nn.LayerNorm modules (or None: no LayerNorm) and
    the q scale; the parameters must be on the device, in `dtype`."""
    if q_norm is None:
        return PrimeQkNorm(None, None, None, None, _DTYPES[dtype], 1e-5, float(q_scale))
    ps = [q_norm.weight, q_norm.bias, k_norm.weight, k_norm.bias]
    for t in ps:
        if t is None or t.dtype != dtype or not t.is_contiguous():
            raise ValueError(f"QK LayerNorm parameters must be contiguous {dtype} with bias")
        _dev_check(t)
    return PrimeQkNorm(*[t.data_ptr() for t in ps], _DTYPES[dtype], float(q_norm.eps), float(q_scale))


def qk_norm_on_load(q_norm, k_norm, q_scale: float, q: torch.Tensor) -> Optional[PrimeQkNorm]:
    """The QK-norm for the bf16 prefill kernels to apply as they load q and k,
    or None where q and k must be normalised first: projections other than
    bf16, LayerNorm parameters of another dtype or device, or q and k
    LayerNorms with different eps (the kernels take one)."""
    if q.dtype != torch.bfloat16:
        return None
    if q_norm is not None:
        ps = (q_norm.weight, q_norm.bias, k_norm.weight, k_norm.bias)
        if any(t is None or t.dtype != q.dtype or not t.is_contiguous() or t.device != q.device for t in ps):
            return None
        if q_norm.eps != k_norm.eps:
            return None
    return qk_norm(q_norm, k_norm, q_scale, q.dtype)


def decode_step_qknorm(q, k, v, decay: torch.Tensor, eps: float, norm: PrimeQkNorm, state_in, state_out,
                       y, y_frag: bool = False) -> None:
    """prime_decode_step_qknorm: q, k the raw projections [B,H,D] / [B,Hkv,D];
    the QK LayerNorm and q scale (``qk_norm(...)``) are applied in the kernel.
    y_frag: y is a flat bf16 buffer receiving the output in the fragment layout."""
    _decode_checks(q, k, v, decay, state_in, state_out, y, y_frag)
    B, H, D = q.shape
    L = load()
    qd, kd, vd, yd = tensor_desc(q, False), tensor_desc(k, False), tensor_desc(v, False), _y_desc(y, B, H, D, y_frag)
    si, so = state_desc(state_in), state_desc(state_out)
    rc = L.prime_decode_step_qknorm(ctypes.byref(qd), ctypes.byref(kd), ctypes.byref(vd), B, H, k.shape[1], D,
                                    decay.data_ptr(), float(eps), ctypes.byref(norm),
                                    ctypes.byref(si) if si else None, ctypes.byref(so), ctypes.byref(yd),
                                    _stream(q.device))
    _check(rc, "prime_decode_step_qknorm")


def add_rmsnorm(x: torch.Tensor, delta: Optional[torch.Tensor], weight: torch.Tensor, out: torch.Tensor,
                eps: float) -> None:
    """prime_add_rmsnorm: x <- x + delta (if delta), out <- RMSNorm(x) * weight;
    x, delta, out contiguous [..., hidden] of one dtype, weight [hidden]."""
    _dev_check(x, weight, out, delta)
    hidden = x.shape[-1]
    for t in (x, out) + ((delta,) if delta is not None else ()):
        if not t.is_contiguous() or t.dtype != x.dtype or t.shape != x.shape:
            raise ValueError("x, delta and out must be contiguous tensors of one shape and dtype")
    if weight.dtype != x.dtype or weight.numel() != hidden or not weight.is_contiguous():
        raise ValueError("weight must be a contiguous [hidden] tensor of x's dtype")
    if x.dtype not in _DTYPES:
        raise RuntimeError(f"unsupported dtype {x.dtype}")
    rows = x.numel() // hidden
    rc = load().prime_add_rmsnorm(ctypes.c_void_p(x.data_ptr()),
                                  ctypes.c_void_p(delta.data_ptr()) if delta is not None else None,
                                  ctypes.c_void_p(weight.data_ptr()), ctypes.c_void_p(out.data_ptr()), rows,
                                  hidden, _DTYPES[x.dtype], float(eps), _stream(x.device))
    _check(rc, "prime_add_rmsnorm")


def gelu(x: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """prime_gelu: out = GELU(x) (exact erf form, fp32 math, one rounding);
    x contiguous; out defaults to x (in place)."""
    if out is None:
        out = x
    _dev_check(x, out)
    if not x.is_contiguous() or not out.is_contiguous() or out.dtype != x.dtype or out.numel() != x.numel():
        raise ValueError("x and out must be contiguous tensors of one size and dtype")
    if x.dtype not in _DTYPES:
        raise RuntimeError(f"unsupported dtype {x.dtype}")
    rc = load().prime_gelu(ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(out.data_ptr()),
                           ctypes.c_int64(x.numel()), _DTYPES[x.dtype], _stream(x.device))
    _check(rc, "prime_gelu")
    return out


def head_layernorm(x: torch.Tensor, out: torch.Tensor, norm: Optional[torch.nn.LayerNorm], scale: float) -> None:
    """prime_head_layernorm: out = round(round(LayerNorm(x)) * scale) per
    [B, H, L, 64] row (norm None: the scale only); out may be x."""
    _dev_check(x, out)
    if x.dim() != 4 or out.shape != x.shape or out.dtype != x.dtype:
        raise ValueError("x and out must be [B, H, L, D] views of one shape and dtype")
    B, H, L, D = x.shape
    w = b = None
    pdt = _DTYPES.get(x.dtype, 0)
    eps = 1e-5
    if norm is not None:
        if norm.weight is None or norm.bias is None:
            raise ValueError("the LayerNorm needs weight and bias")
        w, b, eps = norm.weight, norm.bias, norm.eps
        if w.dtype not in _DTYPES or b.dtype != w.dtype or not (w.is_contiguous() and b.is_contiguous()):
            raise ValueError("LayerNorm parameters must be contiguous and of one supported dtype")
        pdt = _DTYPES[w.dtype]
    xd, od = tensor_desc(x, True), tensor_desc(out, True)
    rc = load().prime_head_layernorm(ctypes.byref(xd), ctypes.byref(od), B, H, L, D,
                                     ctypes.c_void_p(w.data_ptr()) if w is not None else None,
                                     ctypes.c_void_p(b.data_ptr()) if b is not None else None, pdt,
                                     float(eps), float(scale), _stream(x.device))
    _check(rc, "prime_head_layernorm")


EPILOGUE_NONE, EPILOGUE_GELU, EPILOGUE_RESIDUAL = 0, 1, 2


def _linear_checks(x, w, out, who):
    _dev_check(x, w, out)
    if x.dim() != 2 or w.dim() != 2 or out.dim() != 2:
        raise ValueError("x, w and out must be 2-D")
    M, K = x.shape
    N = w.shape[0]
    if w.shape[1] != K or out.shape != (M, N):
        raise ValueError(f"shape mismatch: x {tuple(x.shape)}, w {tuple(w.shape)}, out {tuple(out.shape)}")
    if x.dtype != torch.bfloat16 or w.dtype != torch.bfloat16 or out.dtype != torch.bfloat16:
        raise RuntimeError(f"{who} takes bf16 tensors")
    if x.stride(1) != 1 or w.stride(1) != 1 or out.stride(1) != 1:
        raise ValueError("the last dimension must be contiguous")
    return M, N, K


def linear(x: torch.Tensor, w: torch.Tensor, out: torch.Tensor, epilogue: int = EPILOGUE_NONE) -> torch.Tensor:
    """prime_linear: out = epilogue(x @ w.T) for bf16 x [M, K], w [N, K],
    out [M, N] (rows with a contiguous last dimension); returns out."""
    M, N, K = _linear_checks(x, w, out, "prime_linear")
    rc = load().prime_linear(ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(w.data_ptr()),
                             ctypes.c_void_p(out.data_ptr()), M, N, K, x.stride(0), w.stride(0), out.stride(0),
                             _DTYPES[torch.bfloat16], int(epilogue), _stream(x.device))
    _check(rc, "prime_linear")
    return out


def linear_residual(x: torch.Tensor, w: torch.Tensor, r: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """prime_linear_residual: out = r + x @ w.T (the product rounded to bf16,
    then the add rounded), bf16; r [M, N] may be out itself (in place)."""
    M, N, K = _linear_checks(x, w, out, "prime_linear_residual")
    _dev_check(r)
    if r.shape != (M, N) or r.dtype != torch.bfloat16 or r.stride(1) != 1:
        raise ValueError("r must be a bf16 [M, N] tensor with a contiguous last dimension")
    rc = load().prime_linear_residual(ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(w.data_ptr()),
                                      ctypes.c_void_p(r.data_ptr()), ctypes.c_void_p(out.data_ptr()), M, N, K,
                                      x.stride(0), w.stride(0), r.stride(0), out.stride(0),
                                      _DTYPES[torch.bfloat16], _stream(x.device))
    _check(rc, "prime_linear_residual")
    return out


def linear_fused(x: torch.Tensor, w: torch.Tensor, out: torch.Tensor, epilogue: int = EPILOGUE_NONE,
                 rms_eps: float = 0.0, r: Optional[torch.Tensor] = None) -> torch.Tensor:
    """prime_linear_fused: out = epilogue(s * x @ w.T) for a few hundred bf16
    rows, s = rsqrt(mean(x^2) + rms_eps) per row when rms_eps > 0 (w carrying
    the RMSNorm weight in its columns), epilogue NONE, GELU or RESIDUAL
    (out = r + product; r may be out)."""
    M, N, K = _linear_checks(x, w, out, "prime_linear_fused")
    if epilogue == EPILOGUE_RESIDUAL:
        if r is None:
            raise ValueError("the residual epilogue needs r")
        _dev_check(r)
        if r.shape != (M, N) or r.dtype != torch.bfloat16 or r.stride(1) != 1:
            raise ValueError("r must be a bf16 [M, N] tensor with a contiguous last dimension")
    rp = r.data_ptr() if r is not None else None
    rc = load().prime_linear_fused(ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(w.data_ptr()), ctypes.c_void_p(rp),
                                   ctypes.c_void_p(out.data_ptr()), M, N, K, x.stride(0), w.stride(0),
                                   r.stride(0) if r is not None else N, out.stride(0), _DTYPES[torch.bfloat16],
                                   int(epilogue), float(rms_eps), _stream(x.device))
    _check(rc, "prime_linear_fused")
    return out


def argmax(logits: torch.Tensor, out: torch.Tensor) -> None:
    """prime_argmax: out[i] = argmax_j logits[i, j] (first index of the
    largest, NaN largest), logits [n, vocab] with a contiguous last dimension,
    out int64 [n] (or [n, 1])."""
    _dev_check(logits, out)
    if logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError("logits must be [n, vocab] with a contiguous vocab dimension")
    if logits.dtype not in _DTYPES:
        raise RuntimeError(f"unsupported dtype {logits.dtype}")
    n, vocab = logits.shape
    if out.dtype != torch.int64 or out.numel() != n or not out.is_contiguous():
        raise ValueError("out must be a contiguous int64 tensor of n elements")
    rc = load().prime_argmax(ctypes.c_void_p(logits.data_ptr()), _DTYPES[logits.dtype], n, vocab,
                             logits.stride(0), ctypes.c_void_p(out.data_ptr()), _stream(logits.device))
    _check(rc, "prime_argmax")


def workspace_size(B: int, H: int, L: int, flags: int = 0) -> int:
    return int(load().prime_chunked_prefill_workspace_size(B, H, L, flags))


def _prefill_args(q, k, v, decay, eps, chunk, state_in, y, state_out, flags, workspace):
    _dev_check(q, k, v, y, decay)
    B, H, Lq, D = q.shape
    Hkv = k.shape[1]
    _shape(k, (B, Hkv, Lq, D), "k")
    _shape(v, (B, Hkv, Lq, D), "v")
    _shape(y, (B, H, Lq, D), "y")
    _check_decay(decay, H)
    _check_state(state_in, B, H, D, "state_in")
    _check_state(state_out, B, H, D, "state_out")
    if workspace is None:
        nbytes = workspace_size(B, H, Lq, flags)
        workspace = torch.empty(nbytes, dtype=torch.uint8, device=q.device) if nbytes else None
    elif workspace.numel() == 0:
        workspace = None
    else:
        _dev_check(workspace)
    ws_ptr = workspace.data_ptr() if workspace is not None else None
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    refs = (tensor_desc(q, True), tensor_desc(k, True), tensor_desc(v, True), state_desc(state_in),
            tensor_desc(y, True), state_desc(state_out))
    args = (ctypes.byref(refs[0]), ctypes.byref(refs[1]), ctypes.byref(refs[2]), B, H, Hkv, Lq, D,
            int(chunk), ctypes.c_void_p(decay.data_ptr()), ctypes.c_float(eps), int(flags),
            ctypes.byref(refs[3]) if refs[3] else None, ctypes.byref(refs[4]),
            ctypes.byref(refs[5]) if refs[5] else None, ws_ptr, ws_bytes)
    return args, (q, k, v, decay, state_in, y, state_out, workspace, refs)


def chunked_prefill(q, k, v, decay: torch.Tensor, eps: float, chunk: int, state_in, y,
                    state_out, flags: int = 0, workspace: Optional[torch.Tensor] = None,
                    qk_norm: Optional[PrimeQkNorm] = None) -> None:
    """Chunked prefill (prime_chunked_prefill).  q [B,H,L,D], k/v [B,Hkv,L,D].
    workspace: None allocates the recommended scratch from torch's caching
    allocator; pass an empty tensor to run one segment per sequence.
    qk_norm (``qk_norm(...)``, bf16 only): q, k are the raw projections and the
    module's QK LayerNorm and q scale are applied as the kernels load them
    (prime_chunked_prefill_qknorm)."""
    args, keep = _prefill_args(q, k, v, decay, eps, chunk, state_in, y, state_out, flags, workspace)
    if qk_norm is None:
        _check(load().prime_chunked_prefill(*args, _stream(q.device)), "prime_chunked_prefill")
    else:
        args = args[:12] + (ctypes.byref(qk_norm),) + args[12:]
        _check(load().prime_chunked_prefill_qknorm(*args, _stream(q.device)), "prime_chunked_prefill_qknorm")
    del keep


def _sel_vec(t: torch.Tensor, n: int, name: str) -> None:
    _dev_check(t)
    if t.dtype != torch.float32 or t.numel() != n or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous fp32 tensor of {n} elements")


def selective_log_decay(step: torch.Tensor, tau: torch.Tensor, step_min: float = 1e-4, step_max: float = 50.0,
                        out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """prime_selective_log_decay: -clamp(softplus(step), step_min, step_max) /
    tau as fp32 [B, H, L] (each stage rounded to step's dtype, as the module's
    tensors hold it) from the pre-activations step = delta_proj(x) [B, L, H]
    (any batch and token strides, contiguous heads); tau fp32 [H]."""
    _dev_check(step)
    if step.dim() != 3 or step.stride(2) != 1 or step.dtype not in _DTYPES:
        raise ValueError("step must be [B, L, H] with contiguous heads")
    B, Lt, H = step.shape
    _sel_vec(tau, H, "tau")
    if out is None:
        out = torch.empty(B, H, Lt, device=step.device, dtype=torch.float32)
    elif out.shape != (B, H, Lt) or out.dtype != torch.float32 or not out.is_contiguous():
        raise ValueError("out must be a contiguous fp32 [B, H, L] tensor")
    rc = load().prime_selective_log_decay(ctypes.c_void_p(step.data_ptr()), _DTYPES[step.dtype], step.stride(0),
                                          step.stride(1), ctypes.c_void_p(tau.data_ptr()), float(step_min),
                                          float(step_max), B, H, Lt, ctypes.c_void_p(out.data_ptr()),
                                          _stream(step.device))
    _check(rc, "prime_selective_log_decay")
    return out


def selective_prefill(q, k, v, log_decay: torch.Tensor, k_scale: torch.Tensor, eps: float, state_in, y,
                      state_out, workspace: Optional[torch.Tensor] = None,
                      qk_norm: Optional[PrimeQkNorm] = None) -> None:
    """Selective PRIME prefill (prime_selective_prefill): q [B,H,L,D], k/v
    [B,Hkv,L,D], bf16 (bf16 MFMA operands) or fp32 (an fp32 kernel); log_decay
    fp32 [B,H,L] (log lambda_t, contiguous); k_scale fp32 [H] (beta); states in
    the selective convention.  qk_norm (bf16 only): as for chunked_prefill
    (prime_selective_prefill_qknorm)."""
    B, H, Lq, D = q.shape
    _sel_vec(log_decay, B * H * Lq, "log_decay")
    _sel_vec(k_scale, H, "k_scale")
    # the decay argument of the base form is not used: pass the k scale for the checks
    args, keep = _prefill_args(q, k, v, k_scale, eps, 64, state_in, y, state_out, 0, workspace)
    head = args[:8] + (ctypes.c_void_p(log_decay.data_ptr()), ctypes.c_void_p(k_scale.data_ptr()), args[10])
    if qk_norm is None:
        _check(load().prime_selective_prefill(*(head + args[12:]), _stream(q.device)), "prime_selective_prefill")
    else:
        _check(load().prime_selective_prefill_qknorm(*(head + (ctypes.byref(qk_norm),) + args[12:]),
                                                      _stream(q.device)), "prime_selective_prefill_qknorm")
    del keep


def selective_gate(B: int, H: int, decay_bh: Optional[torch.Tensor] = None, step: Optional[torch.Tensor] = None,
                   tau: Optional[torch.Tensor] = None, step_min: float = 1e-4,
                   step_max: float = 50.0) -> PrimeSelectiveGate:
    """prime_selective_gate_t: lambda_t per (sequence, head) as decay_bh fp32
    [B,H], or the step pre-activations `step` [B,H] (delta_proj(x), any row
    stride, contiguous heads) with tau fp32 [H] (the kernel forms the decays)."""
    if decay_bh is not None:
        _sel_vec(decay_bh, B * H, "decay_bh")
        return PrimeSelectiveGate(decay_bh.data_ptr(), None, 0, 0, 0, None, 0.0, 0.0)
    if step is None or tau is None:
        raise ValueError("give decay_bh, or step and tau")
    _dev_check(step)
    _sel_vec(tau, H, "tau")
    if step.dim() != 2 or step.shape != (B, H) or step.stride(1) != 1 or step.dtype not in _DTYPES:
        raise ValueError("step must be [B, H] with contiguous heads")
    return PrimeSelectiveGate(None, step.data_ptr(), _DTYPES[step.dtype], 0, step.stride(0), tau.data_ptr(),
                              float(step_min), float(step_max))


def selective_decode_step(q, k, v, gate: PrimeSelectiveGate, k_scale: torch.Tensor, eps: float,
                          norm: Optional[PrimeQkNorm], state_in, state_out, y, y_frag: bool = False) -> None:
    """Selective PRIME decode step (prime_selective_decode_step): the decays
    from ``selective_gate(...)``, k_scale fp32 [H]; norm: the QK LayerNorm
    and q scale for raw projections (``qk_norm(...)``) or None.  The tensors
    the gate points to must stay alive until the call returns."""
    B, H, D = q.shape
    _decode_checks(q, k, v, k_scale, state_in, state_out, y, y_frag)
    L = load()
    qd, kd, vd, yd = tensor_desc(q, False), tensor_desc(k, False), tensor_desc(v, False), _y_desc(y, B, H, D, y_frag)
    si, so = state_desc(state_in), state_desc(state_out)
    rc = L.prime_selective_decode_step(ctypes.byref(qd), ctypes.byref(kd), ctypes.byref(vd), B, H, k.shape[1], D,
                                       ctypes.byref(gate), k_scale.data_ptr(), float(eps),
                                       ctypes.byref(norm) if norm is not None else None,
                                       ctypes.byref(si) if si else None, ctypes.byref(so), ctypes.byref(yd),
                                       _stream(q.device))
    _check(rc, "prime_selective_decode_step")


def backward_workspace_size(B: int, H: int, L: int) -> int:
    return int(load().prime_chunked_prefill_backward_workspace_size(B, H, L))


def chunked_prefill_backward(q, k, v, decay: torch.Tensor, eps: float, state_in, dy, dstate_out, dq, dk, dv,
                             dstate_in, flags: int = 0, workspace: Optional[torch.Tensor] = None) -> None:
    """Backward of the chunked prefill (prime_chunked_prefill_backward).
    q, k, v [B,H,L,D] (bf16 or fp32, k/v with H heads), dy [B,H,L,D];
    dstate_out / state_in / dstate_in: 6-tuples or None; dq, dk, dv share a
    dtype and strides."""
    _dev_check(q, k, v, dy, dq, dk, dv, decay)
    B, H, Lq, D = q.shape
    for t, n in ((k, "k"), (v, "v"), (dy, "dy"), (dq, "dq"), (dk, "dk"), (dv, "dv")):
        _shape(t, (B, H, Lq, D), n)
    _check_decay(decay, H)
    _check_state(state_in, B, H, D, "state_in")
    _check_state(dstate_out, B, H, D, "dstate_out")
    _check_state(dstate_in, B, H, D, "dstate_in")
    if workspace is None:
        workspace = torch.empty(max(backward_workspace_size(B, H, Lq), 4), dtype=torch.uint8, device=q.device)
    descs = [tensor_desc(t, True) for t in (q, k, v, dy, dq, dk, dv)]
    si, so, sd = state_desc(state_in), state_desc(dstate_out), state_desc(dstate_in)
    r = lambda x: ctypes.byref(x) if x is not None else None
    rc = load().prime_chunked_prefill_backward(
        r(descs[0]), r(descs[1]), r(descs[2]), B, H, H, Lq, D, decay.data_ptr(), float(eps), int(flags), r(si),
        r(descs[3]), r(so), r(descs[4]), r(descs[5]), r(descs[6]), r(sd), workspace.data_ptr(),
        workspace.numel() * workspace.element_size(), _stream(q.device))
    _check(rc, "prime_chunked_prefill_backward")


def selective_backward_workspace_size(B: int, H: int, L: int) -> int:
    return int(load().prime_selective_prefill_backward_workspace_size(B, H, L))


def selective_prefill_backward(q, k, v, log_decay: torch.Tensor, k_scale: torch.Tensor, eps: float, state_in, dy,
                               dstate_out, dq, dk, dv, dstate_in, d_log_decay: torch.Tensor,
                               d_k_scale: torch.Tensor, workspace: Optional[torch.Tensor] = None) -> None:
    """Backward of the selective prefill (prime_selective_prefill_backward).
    q, k, v [B,H,L,D] fp32 (k/v with H heads), dy [B,H,L,D]; log_decay fp32
    [B,H,L]; k_scale fp32 [H]; states (selective convention) 6-tuples or
    None; outputs dq/dk/dv (one dtype and stride set), dstate_in,
    d_log_decay fp32 [B,H,L] and d_k_scale fp32 [B,H] (per sequence)."""
    _dev_check(q, k, v, dy, dq, dk, dv, log_decay, k_scale, d_log_decay, d_k_scale)
    B, H, Lq, D = q.shape
    for t, n in ((k, "k"), (v, "v"), (dy, "dy"), (dq, "dq"), (dk, "dk"), (dv, "dv")):
        _shape(t, (B, H, Lq, D), n)
    _sel_vec(log_decay, B * H * Lq, "log_decay")
    _sel_vec(k_scale, H, "k_scale")
    _sel_vec(d_log_decay, B * H * Lq, "d_log_decay")
    _sel_vec(d_k_scale, B * H, "d_k_scale")
    _check_state(state_in, B, H, D, "state_in")
    _check_state(dstate_out, B, H, D, "dstate_out")
    _check_state(dstate_in, B, H, D, "dstate_in")
    if workspace is None:
        workspace = torch.empty(max(selective_backward_workspace_size(B, H, Lq), 4), dtype=torch.uint8,
                                device=q.device)
    descs = [tensor_desc(t, True) for t in (q, k, v, dy, dq, dk, dv)]
    si, so, sd = state_desc(state_in), state_desc(dstate_out), state_desc(dstate_in)
    r = lambda x: ctypes.byref(x) if x is not None else None
    rc = load().prime_selective_prefill_backward(
        r(descs[0]), r(descs[1]), r(descs[2]), B, H, H, Lq, D, log_decay.data_ptr(), k_scale.data_ptr(),
        float(eps), r(si), r(descs[3]), r(so), r(descs[4]), r(descs[5]), r(descs[6]), r(sd),
        d_log_decay.data_ptr(), d_k_scale.data_ptr(), workspace.data_ptr(),
        workspace.numel() * workspace.element_size(), _stream(q.device))
    _check(rc, "prime_selective_prefill_backward")


def accumulate_workspace_size(B: int, H: int, L: int) -> int:
    return int(load().prime_accumulate_workspace_size(B, H, L))


def _accumulate_checks(k, v, decay, state_in, state_out, H):
    _dev_check(k, v, decay)
    B, Hkv, Lk, D = k.shape
    H = Hkv if H is None else H
    _shape(v, (B, Hkv, Lk, D), "v")
    _check_decay(decay, H)
    _check_state(state_in, B, H, D, "state_in")
    _check_state(state_out, B, H, D, "state_out")
    return B, H, Hkv, Lk, D


def accumulate(k, v, decay: torch.Tensor, state_in, state_out, H: Optional[int] = None,
               workspace: Optional[torch.Tensor] = None) -> None:
    """State of the tokens of k/v [B,Hkv,L,D] (prime_accumulate), appended to
    state_in (None: zeros) and written to state_out (may be state_in).  H
    query heads (default Hkv; a multiple of Hkv)."""
    B, H, Hkv, Lk, D = _accumulate_checks(k, v, decay, state_in, state_out, H)
    if workspace is None:
        workspace = torch.empty(max(accumulate_workspace_size(B, H, Lk), 1), dtype=torch.uint8, device=k.device)
    _dev_check(workspace)
    kd, vd = tensor_desc(k, True), tensor_desc(v, True)
    si, so = state_desc(state_in), state_desc(state_out)
    rc = load().prime_accumulate(ctypes.byref(kd), ctypes.byref(vd), B, H, Hkv, Lk, D, decay.data_ptr(),
                                 ctypes.byref(si) if si else None, ctypes.byref(so), workspace.data_ptr(),
                                 workspace.numel() * workspace.element_size(), _stream(k.device))
    _check(rc, "prime_accumulate")


def accumulate_noalloc(k, v, decay: torch.Tensor, state_in, state_out, H: Optional[int] = None) -> None:
    """accumulate() through prime_accumulate_noalloc: no workspace, nothing
    allocated (the segment slots live in the library's fixed device scratch
    of NOALLOC_SCRATCH_BYTES; B * H at most 992).  Calls that overlap on one
    device share that scratch."""
    B, H, Hkv, Lk, D = _accumulate_checks(k, v, decay, state_in, state_out, H)
    kd, vd = tensor_desc(k, True), tensor_desc(v, True)
    si, so = state_desc(state_in), state_desc(state_out)
    rc = load().prime_accumulate_noalloc(ctypes.byref(kd), ctypes.byref(vd), B, H, Hkv, Lk, D, decay.data_ptr(),
                                         ctypes.byref(si) if si else None, ctypes.byref(so), _stream(k.device))
    _check(rc, "prime_accumulate_noalloc")


def decode_readout(q, eps: float, state, y) -> None:
    """y = the moment readout of q [B,H,D] against `state` (prime_decode_readout)."""
    _dev_check(q, y)
    B, H, D = q.shape
    _shape(y, (B, H, D), "y")
    _check_state(state, B, H, D, "state")
    qd, yd, sd = tensor_desc(q, False), tensor_desc(y, False), state_desc(state)
    rc = load().prime_decode_readout(ctypes.byref(qd), B, H, D, float(eps), ctypes.byref(sd), ctypes.byref(yd),
                                     _stream(q.device))
    _check(rc, "prime_decode_readout")


def decode_update(k, v, decay: torch.Tensor, state_in, state_out, H: Optional[int] = None) -> None:
    """Append one token of k/v [B,Hkv,D] to the state (prime_decode_update)."""
    _dev_check(k, v, decay)
    B, Hkv, D = k.shape
    H = Hkv if H is None else H
    _shape(v, (B, Hkv, D), "v")
    _check_decay(decay, H)
    _check_state(state_in, B, H, D, "state_in")
    _check_state(state_out, B, H, D, "state_out")
    kd, vd = tensor_desc(k, False), tensor_desc(v, False)
    si, so = state_desc(state_in), state_desc(state_out)
    rc = load().prime_decode_update(ctypes.byref(kd), ctypes.byref(vd), B, H, Hkv, D, decay.data_ptr(),
                                    ctypes.byref(si) if si else None, ctypes.byref(so), _stream(k.device))
    _check(rc, "prime_decode_update")


def bind_chunked_prefill(q, k, v, decay: torch.Tensor, eps: float, chunk: int, state_in, y,
                         state_out, flags: int = 0, workspace: Optional[torch.Tensor] = None):
    """Validate once and return a no-argument callable that launches
    prime_chunked_prefill on these exact buffers (current stream at call time);
    the workspace, if allocated here, is held by the callable."""
    args, keep = _prefill_args(q, k, v, decay, eps, chunk, state_in, y, state_out, flags, workspace)
    fn, dev = load().prime_chunked_prefill, q.device

    def launch():
        _check(fn(*args, torch.cuda.current_stream(dev).cuda_stream), "prime_chunked_prefill")
    launch.buffers = keep
    return launch


# ---------------------------------------------------------------- delta rule
def _check_delta_state(S, B, H, D, name):
    if S is None:
        return
    if S.dtype != torch.float32 or not S.is_contiguous() or S.numel() != B * H * D * 2 * D:
        raise ValueError(f"{name} must be a contiguous fp32 [B, H, D, 2D] tensor")
    _dev_check(S)


def _gate(t, B, H, L, name):
    if t.dtype != torch.float32 or not t.is_contiguous() or t.numel() != B * H * L:
        raise ValueError(f"{name} must be a contiguous fp32 tensor of {B * H * L} values ([B, H, L])")
    _dev_check(t)


PRIME_FLAG_F32_INPUTS = 2


def delta_workspace_size(B: int, H: int, L: int, dtype=None) -> int:
    """Workspace bytes of prime_delta_prefill; fp32 inputs (``dtype`` torch.float32)
    need records twice the size of bf16 inputs'."""
    flags = PRIME_FLAG_F32_INPUTS if dtype == torch.float32 else 0
    return int(load().prime_delta_prefill_workspace_size(B, H, L, flags))


def delta_generic(D: int, chunk: int) -> bool:
    """True for the shapes the token-sequential delta kernels run (any head dim
    up to 64 and chunk other than D = 64 with chunk 64)."""
    return D != 64 or chunk != 64


def delta_prefill(q, k, v, beta, alpha, decay_pad: float, feat_eps: float, bound: float, state_in, y,
                  state_out, workspace: Optional[torch.Tensor] = None, chunk: int = 64) -> None:
    """Chunked delta-rule prefill (prime_delta_prefill).  q [B,H,L,D], k/v
    [B,Hkv,L,D] (bf16 or fp32 alike at D = 64, chunk 64; any supported dtypes
    otherwise), beta/alpha fp32 [B,H,L], states fp32 [B,H,D,2D] or None, y
    [B,H,L,D]; the Lyapunov clamp per `chunk` tokens.  workspace None
    allocates the recommended size from torch's caching allocator (none is
    needed outside D = 64 with chunk 64)."""
    _dev_check(q, k, v, y)
    B, H, Lq, D = q.shape
    Hkv = k.shape[1]
    _shape(k, (B, Hkv, Lq, D), "k")
    _shape(v, (B, Hkv, Lq, D), "v")
    _shape(y, (B, H, Lq, D), "y")
    _gate(beta, B, H, Lq, "beta")
    _gate(alpha, B, H, Lq, "alpha")
    _check_delta_state(state_in, B, H, D, "state_in")
    _check_delta_state(state_out, B, H, D, "state_out")
    if workspace is None and not delta_generic(D, chunk):
        workspace = torch.empty(delta_workspace_size(B, H, Lq, q.dtype), dtype=torch.uint8, device=q.device)
    if workspace is not None:
        _dev_check(workspace)
    qd, kd, vd, yd = tensor_desc(q, True), tensor_desc(k, True), tensor_desc(v, True), tensor_desc(y, True)
    ptr = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else None
    rc = load().prime_delta_prefill(ctypes.byref(qd), ctypes.byref(kd), ctypes.byref(vd), ptr(beta), ptr(alpha),
                                    B, H, Hkv, Lq, D, int(chunk), float(decay_pad), float(feat_eps), float(bound),
                                    ptr(state_in), ctypes.byref(yd), ptr(state_out), ptr(workspace),
                                    workspace.numel() if workspace is not None else 0, _stream(q.device))
    _check(rc, "prime_delta_prefill")


def delta_backward_workspace_size(B: int, H: int, L: int, D: int = 64, chunk: int = 64) -> int:
    return int(load().prime_delta_prefill_backward_workspace_size(B, H, L, D, chunk))


def delta_prefill_backward(q, k, v, beta, alpha, decay_pad: float, feat_eps: float, bound: float, state_in, dy,
                           dstate_out, workspace: Optional[torch.Tensor] = None, chunk: int = 64):
    """Gradients of the chunked delta-rule prefill (prime_delta_prefill_backward)
    for the forward's inputs: returns (dq [B,H,L,D], dk, dv [B,Hkv,L,D] summed
    over each group of query heads, dbeta, dalpha [B,H,L], dstate_in [B,H,D,2D]
    or None when state_in is None), all fp32."""
    _dev_check(q, k, v, dy)
    B, H, Lq, D = q.shape
    Hkv = k.shape[1]
    _shape(k, (B, Hkv, Lq, D), "k")
    _shape(v, (B, Hkv, Lq, D), "v")
    _shape(dy, (B, H, Lq, D), "dy")
    _gate(beta, B, H, Lq, "beta")
    _gate(alpha, B, H, Lq, "alpha")
    _check_delta_state(state_in, B, H, D, "state_in")
    _check_delta_state(dstate_out, B, H, D, "dstate_out")
    dev = q.device
    f32 = dict(device=dev, dtype=torch.float32)
    dq = torch.empty(B, H, Lq, D, **f32)
    dk = torch.empty(B, H, Lq, D, **f32)
    dv = torch.empty(B, H, Lq, D, **f32)
    dbeta = torch.empty(B, H, Lq, **f32)
    dalpha = torch.empty(B, H, Lq, **f32)
    dstate = torch.empty(B, H, D, 2 * D, **f32) if state_in is not None else None
    if workspace is None:
        workspace = torch.empty(delta_backward_workspace_size(B, H, Lq, D, chunk), dtype=torch.uint8, device=dev)
    qd, kd, vd, yd = tensor_desc(q, True), tensor_desc(k, True), tensor_desc(v, True), tensor_desc(dy, True)
    ptr = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else None
    rc = load().prime_delta_prefill_backward(
        ctypes.byref(qd), ctypes.byref(kd), ctypes.byref(vd), ptr(beta), ptr(alpha), B, H, Hkv, Lq, D, int(chunk),
        float(decay_pad), float(feat_eps), float(bound), ptr(state_in), ctypes.byref(yd), ptr(dstate_out), ptr(dq),
        ptr(dk), ptr(dv), ptr(dbeta), ptr(dalpha), ptr(dstate), ptr(workspace),
        workspace.numel() * workspace.element_size(), _stream(dev))
    _check(rc, "prime_delta_prefill_backward")
    if Hkv != H:
        dk = dk.view(B, Hkv, H // Hkv, Lq, D).sum(2)
        dv = dv.view(B, Hkv, H // Hkv, Lq, D).sum(2)
    return dq, dk, dv, dbeta, dalpha, dstate


def delta_decode_step(q, k, v, beta, alpha, feat_eps: float, bound: float, state_in, state_out, y) -> None:
    """One delta-rule decode step (prime_delta_decode_step).  q [B,H,D], k/v
    [B,Hkv,D], beta/alpha fp32 [B,H], states fp32 [B,H,D,2D] (state_in None:
    zero), y [B,H,D]."""
    _dev_check(q, k, v, y)
    B, H, D = q.shape
    Hkv = k.shape[1]
    _shape(k, (B, Hkv, D), "k")
    _shape(v, (B, Hkv, D), "v")
    _shape(y, (B, H, D), "y")
    _gate(beta, B, H, 1, "beta")
    _gate(alpha, B, H, 1, "alpha")
    _check_delta_state(state_in, B, H, D, "state_in")
    _check_delta_state(state_out, B, H, D, "state_out")
    if state_out is None:
        raise ValueError("state_out is required")
    qd, kd, vd, yd = tensor_desc(q, False), tensor_desc(k, False), tensor_desc(v, False), tensor_desc(y, False)
    ptr = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else None
    rc = load().prime_delta_decode_step(ctypes.byref(qd), ctypes.byref(kd), ctypes.byref(vd), ptr(beta), ptr(alpha),
                                        B, H, Hkv, D, float(feat_eps), float(bound), ptr(state_in), ptr(state_out),
                                        ctypes.byref(yd), _stream(q.device))
    _check(rc, "prime_delta_decode_step")


def delta_decode_step_backward(q, k, v, beta, alpha, feat_eps: float, bound: float, state_in, dy, dstate_out):
    """Gradients of one delta-rule decode step (prime_delta_decode_step_backward)
    for its inputs: returns (dq [B,H,D], dk, dv [B,Hkv,D] summed over each group
    of query heads, dbeta, dalpha [B,H], dstate_in [B,H,D,2D] or None when
    state_in is None), all fp32."""
    _dev_check(q, k, v, dy)
    B, H, D = q.shape
    Hkv = k.shape[1]
    _shape(k, (B, Hkv, D), "k")
    _shape(v, (B, Hkv, D), "v")
    _shape(dy, (B, H, D), "dy")
    _gate(beta, B, H, 1, "beta")
    _gate(alpha, B, H, 1, "alpha")
    _check_delta_state(state_in, B, H, D, "state_in")
    _check_delta_state(dstate_out, B, H, D, "dstate_out")
    f32 = dict(device=q.device, dtype=torch.float32)
    dq = torch.empty(B, H, D, **f32)
    dk = torch.empty(B, H, D, **f32)
    dv = torch.empty(B, H, D, **f32)
    dbeta = torch.empty(B, H, **f32)
    dalpha = torch.empty(B, H, **f32)
    dstate = torch.empty(B, H, D, 2 * D, **f32) if state_in is not None else None
    qd, kd, vd, yd = tensor_desc(q, False), tensor_desc(k, False), tensor_desc(v, False), tensor_desc(dy, False)
    ptr = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else None
    rc = load().prime_delta_decode_step_backward(
        ctypes.byref(qd), ctypes.byref(kd), ctypes.byref(vd), ptr(beta), ptr(alpha), B, H, Hkv, D, float(feat_eps),
        float(bound), ptr(state_in), ctypes.byref(yd), ptr(dstate_out), ptr(dq), ptr(dk), ptr(dv), ptr(dbeta),
        ptr(dalpha), ptr(dstate), _stream(q.device))
    _check(rc, "prime_delta_decode_step_backward")
    if Hkv != H:
        dk = dk.view(B, Hkv, H // Hkv, D).sum(2)
        dv = dv.view(B, Hkv, H // Hkv, D).sum(2)
    return dq, dk, dv, dbeta, dalpha, dstate


def timer_enable(*kernels: int) -> None:
    """Bracket every launch of the given kernels (KERNEL_*) with HIP events;
    no arguments disables the timer (prime_timer_enable)."""
    mask = 0
    for kid in kernels:
        mask |= 1 << kid
    load().prime_timer_enable(mask)


def timer_reset() -> None:
    _check(load().prime_timer_reset(), "prime_timer_reset")


def timer_read(kernel: int) -> Tuple[float, int]:
    """(summed device ms, launches) of one kernel since the last reset."""
    ms, n = ctypes.c_double(), ctypes.c_int64()
    _check(load().prime_timer_read(kernel, ctypes.byref(ms), ctypes.byref(n)), "prime_timer_read")
    return ms.value, n.value


def hbm_stream(src: torch.Tensor, dst: torch.Tensor, copy: bool = True, blocks: int = 0) -> None:
    """prime_hbm_stream: nontemporal 16-byte copy of src into dst (copy), or a
    read-only pass over src (dst receives one 16-byte word per workgroup)."""
    if not (src.is_cuda and dst.is_cuda and src.is_contiguous() and dst.is_contiguous()):
        raise ValueError("hbm_stream: contiguous device tensors")
    nbytes = src.numel() * src.element_size()
    if blocks <= 0:
        blocks = 8 * torch.cuda.get_device_properties(src.device).multi_processor_count
    if copy and dst.numel() * dst.element_size() < nbytes:
        raise ValueError("hbm_stream: dst smaller than src")
    if not copy and dst.numel() * dst.element_size() < 16 * blocks:
        raise ValueError("hbm_stream: dst must hold 16 bytes per workgroup")
    _check(load().prime_hbm_stream(ctypes.c_void_p(src.data_ptr()), ctypes.c_void_p(dst.data_ptr()), nbytes,
                                   1 if copy else 0, blocks, _stream(src.device)), "prime_hbm_stream")


LINEAR_RMS, LINEAR_OUT_FRAG = 1, 2


def frag_rows(M: int) -> int:
    """Rows of the fragment layout of an M-row matrix (M rounded up to 32)."""
    return (M + 31) // 32 * 32


def frag_supported(K: int) -> bool:
    """prime_linear_frag's contraction sizes: 256 x {1, 2, 3, 4, 6, 12}."""
    return K % 256 == 0 and K // 256 in (1, 2, 3, 4, 6, 12)


def pack_frag(src: torch.Tensor, out: Optional[torch.Tensor] = None, rows: Optional[torch.Tensor] = None,
              M: Optional[int] = None) -> torch.Tensor:
    """prime_pack_frag: the bf16 matrix src [R, K] (contiguous rows) in the
    fragment layout, as a flat tensor of frag_rows(M) * K elements; with rows
    (int64 [M] on the device) row r is src[rows[r]] (an embedding gather)."""
    _dev_check(src)
    if src.dim() != 2 or src.dtype != torch.bfloat16 or src.stride(1) != 1:
        raise ValueError("src must be a bf16 [R, K] tensor with contiguous rows")
    R, K = src.shape
    if rows is not None:
        _dev_check(rows)
        if rows.dtype != torch.int64 or not rows.is_contiguous():
            raise ValueError("rows must be a contiguous int64 tensor")
        M = rows.numel()
    M = R if M is None else M
    n = frag_rows(M) * K
    if out is None:
        out = torch.empty(n, device=src.device, dtype=torch.bfloat16)
    elif out.numel() < n or out.dtype != torch.bfloat16 or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous bf16 tensor of at least {n} elements")
    rc = load().prime_pack_frag(ctypes.c_void_p(src.data_ptr()), src.stride(0), R,
                                ctypes.c_void_p(rows.data_ptr()) if rows is not None else None, M, K,
                                ctypes.c_void_p(out.data_ptr()), _stream(src.device))
    _check(rc, "prime_pack_frag")
    return out


def linear_frag_workspace_size(M: int, N: int, K: int) -> int:
    return int(load().prime_linear_frag_workspace_size(M, N, K))


def linear_frag(x: torch.Tensor, w: torch.Tensor, M: int, N: int, K: int, y: Optional[torch.Tensor],
                epilogue: int = EPILOGUE_NONE, flags: int = 0, rms_eps: float = 0.0,
                bias: Optional[torch.Tensor] = None, r: Optional[torch.Tensor] = None, ldy: int = 0,
                tokens: Optional[torch.Tensor] = None, workspace: Optional[torch.Tensor] = None) -> None:
    """prime_linear_frag: y = epilogue(s * x w^T + bias) with x, w in the
    fragment layout (flat bf16 tensors from pack_frag or an earlier
    linear_frag); y row-major [M, ldy] (ldy 0: N) or, with LINEAR_OUT_FRAG,
    fragment layout; tokens (int64 [M]): the argmax of each row's rounded
    products (needs workspace of linear_frag_workspace_size bytes)."""
    _dev_check(x, w, y, bias, r, tokens, workspace)
    Mp = frag_rows(M)
    if x.numel() < Mp * K or w.numel() < N * K or x.dtype != torch.bfloat16 or w.dtype != torch.bfloat16:
        raise ValueError("x and w must be bf16 fragment-layout buffers of frag_rows(M) x K and N x K")
    ldy = ldy or N
    if y is not None:
        need = Mp * N if flags & LINEAR_OUT_FRAG else (M - 1) * ldy + N
        if y.dtype != torch.bfloat16 or y.numel() < need or not y.is_contiguous():
            raise ValueError(f"y must be a contiguous bf16 tensor of at least {need} elements")
    if r is not None:
        need = Mp * N if flags & LINEAR_OUT_FRAG else (M - 1) * ldy + N
        if r.dtype != torch.bfloat16 or not r.is_contiguous() or r.numel() < need:
            raise ValueError(f"r must be a contiguous bf16 tensor in y's layout ({need} elements)")
    if bias is not None and (bias.dtype != torch.float32 or bias.numel() != N or not bias.is_contiguous()):
        raise ValueError(f"bias must be a contiguous fp32 tensor of {N} values")
    if tokens is not None and (tokens.dtype != torch.int64 or tokens.numel() < M):
        raise ValueError("tokens must be an int64 tensor of M values")
    p = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else None
    rc = load().prime_linear_frag(p(x), p(w), p(r), p(y), M, N, K, ldy, int(epilogue), int(flags), float(rms_eps),
                                  p(bias), p(tokens), p(workspace),
                                  workspace.numel() * workspace.element_size() if workspace is not None else 0,
                                  _stream(x.device))
    _check(rc, "prime_linear_frag")


_decay_cache = {}


def decay_tensor(decay, H: int, device: torch.device) -> torch.Tensor:
    """fp32 [H] device tensor for a scalar decay or a per-head tensor."""
    if torch.is_tensor(decay):
        d = decay.detach().to(device=device, dtype=torch.float32).reshape(-1)
        if d.numel() == 1:
            d = d.expand(H)
        if d.numel() != H:
            raise ValueError(f"decay has {d.numel()} values for {H} heads")
        return d.contiguous()
    key = (float(decay), H, str(device))
    t = _decay_cache.get(key)
    if t is None:
        t = torch.full((H,), float(decay), dtype=torch.float32, device=device)
        _decay_cache[key] = t
    return t


def new_state(B: int, H: int, D: int, device, zero: bool = False) -> Tuple[torch.Tensor, ...]:
    f = torch.zeros if zero else torch.empty
    kw = dict(device=device, dtype=torch.float32)
    return (f(B, H, D, **kw), f(B, H, D, D, **kw), f(B, H, D, D, **kw),
            f(B, H, 1, **kw), f(B, H, D, **kw), f(B, H, D, **kw))


def as_state(state, B: int, H: int, D: int, device) -> Tuple[torch.Tensor, ...]:
    """Validate a reference-layout 6-tuple; return contiguous fp32 tensors."""
    if len(state) != 6:
        raise ValueError("state must be the 6-tuple (S0, S1, S2, K0, K1, K2)")
    shapes = [(B, H, D), (B, H, D, D), (B, H, D, D), (B, H, 1), (B, H, D), (B, H, D)]
    out = []
    for t, s in zip(state, shapes):
        if t.numel() != _prod(s):
            raise ValueError(f"state component has shape {tuple(t.shape)}, expected {s}")
        t = t.to(device=device, dtype=torch.float32)
        out.append(t.reshape(s).contiguous())
    return tuple(out)


def _prod(s):
    p = 1
    for x in s:
        p *= x
    return p

"""ctypes binding of the C ABI in include/d2p_amd.h (libd2p_amd.so).

GPU parity tests call the kernels through this boundary with device buffers
owned by torch; no torch types cross it.
"""
import ctypes
import os

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(ROOT, "d2p_amd", "libd2p_amd.so")
HEADER = os.path.join(ROOT, "include", "d2p_amd.h")

_p = ctypes.c_void_p
_i = ctypes.c_int
_f = ctypes.c_float
_z = ctypes.c_size_t
_ll = ctypes.c_longlong

SIGNATURES = {
    "d2p_last_error": (ctypes.c_char_p, []),
    "d2p_abi_version": (_i, []),
    "d2p_sw_workspace_bytes": (_z, [_i, _i, _i]),
    "d2p_sw_forward_marginals": (_i, [_p, _p, _i, _i, _i, _f, _f, _p, _p, _p, _p, _p, _z, _p]),
    "d2p_sw_status": (_i, [_p, _i, ctypes.POINTER(_i), _p]),
    "d2p_sw_forward_marginals_noalloc": (_i, [_p, _p, _i, _i, _i, _f, _f, _p, _p, _p, _p, _p]),
    "d2p_sw_noalloc_scratch_bytes": (_z, []),
    "d2p_set_spin_limit": (_i, [_i]),
    "d2p_swa_workspace_bytes": (_z, [_i, _i, _i]),
    "d2p_swa_forward_marginals": (_i, [_p, _p, _i, _i, _i, _f, _f, _f, _p, _p, _p, _p, _p, _p,
                                       _z, _p]),
    "d2p_nw_workspace_bytes": (_z, [_i, _i, _i]),
    "d2p_nw_forward_marginals": (_i, [_p, _p, _i, _i, _i, _f, _f, _p, _p, _p, _p, _p, _z, _p]),
    "d2p_dtw_workspace_bytes": (_z, [_i, _i, _i]),
    "d2p_dtw_workspace_bytes_banded": (_z, [_i, _i, _i, _i]),
    "d2p_dtw_forward_marginals": (_i, [_p, _p, _i, _i, _i, _f, _i, _p, _p, _p, _p, _z, _p]),
    "d2p_sw_second_workspace_bytes": (_z, [_i, _i, _i]),
    "d2p_sw_hvp": (_i, [_p, _p, _p, _i, _i, _i, _f, _f, _p, _p, _z, _p]),
    "d2p_sw_param_jacobian": (_i, [_p, _i, _p, _i, _i, _i, _f, _f, _p, _p, _z, _p]),
    "d2p_sw_backward_full": (_i, [_p, _p, _p, _i, _i, _i, _f, _f, _p, _p, _p, _p, _z, _p]),
    "d2p_nw_second_workspace_bytes": (_z, [_i, _i, _i]),
    "d2p_nw_hvp": (_i, [_p, _p, _p, _i, _i, _i, _f, _f, _p, _p, _z, _p]),
    "d2p_nw_param_jacobian": (_i, [_p, _i, _p, _i, _i, _i, _f, _f, _p, _p, _z, _p]),
    "d2p_nw_backward_full": (_i, [_p, _p, _p, _i, _i, _i, _f, _f, _p, _p, _p, _p, _z, _p]),
    "d2p_swa_second_workspace_bytes": (_z, [_i, _i, _i]),
    "d2p_swa_hvp": (_i, [_p, _p, _p, _i, _i, _i, _f, _f, _f, _p, _p, _z, _p]),
    "d2p_swa_param_jacobian": (_i, [_p, _i, _p, _i, _i, _i, _f, _f, _f, _p, _p, _z, _p]),
    "d2p_swa_backward_full": (_i, [_p, _p, _p, _i, _i, _i, _f, _f, _f, _p, _p, _p, _p, _p, _z,
                                   _p]),
    "d2p_nwa_workspace_bytes": (_z, [_i, _i, _i]),
    "d2p_nwa_forward_marginals": (_i, [_p, _p, _i, _i, _i, _f, _f, _f, _p, _p, _p, _p, _p, _p,
                                       _z, _p]),
    "d2p_nwa_second_workspace_bytes": (_z, [_i, _i, _i]),
    "d2p_nwa_hvp": (_i, [_p, _p, _p, _i, _i, _i, _f, _f, _f, _p, _p, _z, _p]),
    "d2p_nwa_param_jacobian": (_i, [_p, _i, _p, _i, _i, _i, _f, _f, _f, _p, _p, _z, _p]),
    "d2p_nwa_backward_full": (_i, [_p, _p, _p, _i, _i, _i, _f, _f, _f, _p, _p, _p, _p, _p, _z,
                                   _p]),
    "d2p_dtw_sqeuclid_forward_marginals": (_i, [_p, _p, _p, _i, _i, _i, _i, _f, _i, _p, _p,
                                                _p, _p, _z, _p]),
    "d2p_pairwise_sqdist": (_i, [_p, _p, _i, _i, _i, _i, _p, _p]),
    "d2p_sqeuclid_feature_grad": (_i, [_p, _p, _p, _p, _i, _i, _i, _i, _p, _p, _p]),
    "d2p_dtw_second_workspace_bytes": (_z, [_i, _i, _i]),
    "d2p_dtw_second_workspace_bytes_banded": (_z, [_i, _i, _i, _i]),
    "d2p_dtw_hvp": (_i, [_p, _p, _p, _i, _i, _i, _f, _i, _p, _p, _z, _p]),
    "d2p_dtw_param_jacobian": (_i, [_p, _p, _i, _i, _i, _f, _i, _p, _p, _z, _p]),
    "d2p_dtw_backward_full": (_i, [_p, _p, _p, _i, _i, _i, _f, _i, _p, _p, _p, _z, _p]),
    "d2p_profile_enable": (_i, [_i]),
    "d2p_profile_report": (_i, [ctypes.c_char_p, _z]),
    "d2p_profile_reset": (None, []),
    "d2p_scale_by_batch": (_i, [_p, _p, _p, _i, _ll, _p]),
    "d2p_scale_by_batch_strided": (_i, [_p, _p, _ll, _p, _i, _ll, _p]),
    "d2p_scale_by_batch_lengths": (_i, [_p, _p, _ll, _p, _p, _i, _i, _i, _p]),
}

_lib = None


def lib():
    global _lib
    if _lib is None:
        _lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(_lib, name)
            fn.restype = res
            fn.argtypes = args
    return _lib


def check(rc):
    if rc != 0:
        raise RuntimeError(f"d2p C ABI call failed ({rc}): {lib().d2p_last_error().decode()}")


def ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def stream():
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def sw_forward_marginals(scores, lengths, gap, T):
    """Returns (partition, marginals, grad_gap, grad_T) computed through the C ABI."""
    import torch
    B, L1, L2 = scores.shape
    dev = scores.device
    if lengths is None:
        lengths = torch.tensor([[L1, L2]] * B, dtype=torch.int32, device=dev)
    lengths = lengths.to(dev, torch.int32).contiguous()
    part = torch.empty(B, device=dev)
    marg = torch.empty(B, L1, L2, device=dev)
    gg = torch.empty(B, device=dev)
    gt = torch.empty(B, device=dev)
    nbytes = lib().d2p_sw_workspace_bytes(B, L1, L2)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    check(lib().d2p_sw_forward_marginals(ptr(scores), ptr(lengths), B, L1, L2, gap, T,
                                         ptr(part), ptr(marg), ptr(gg), ptr(gt), ptr(ws),
                                         nbytes, stream()))
    st = ctypes.c_int(0)
    check(lib().d2p_sw_status(ptr(ws), B, ctypes.byref(st), stream()))
    assert st.value == 0, f"pipeline status {st.value}: a stripe wait hit its spin bound"
    return part, marg, gg, gt


def _lengths(lengths, B, L1, L2, dev):
    import torch
    if lengths is None:
        lengths = torch.tensor([[L1, L2]] * B, dtype=torch.int32, device=dev)
    return lengths.to(dev, torch.int32).contiguous()


def _workspace(nbytes, dev):
    import torch
    return torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)


def _check_status(ws, B):
    st = ctypes.c_int(0)
    check(lib().d2p_sw_status(ptr(ws), B, ctypes.byref(st), stream()))
    assert st.value == 0, f"pipeline status {st.value}: a stripe wait hit its spin bound"


def nw_forward_marginals(scores, lengths, gap, T):
    """Linear-gap NW: (value, marginals, grad_gap, grad_T) through the C ABI."""
    import torch
    B, L1, L2 = scores.shape
    dev = scores.device
    lengths = _lengths(lengths, B, L1, L2, dev)
    outs = [torch.empty(B, device=dev), torch.empty(B, L1, L2, device=dev),
            torch.empty(B, device=dev), torch.empty(B, device=dev)]
    nbytes = lib().d2p_nw_workspace_bytes(B, L1, L2)
    ws = _workspace(nbytes, dev)
    check(lib().d2p_nw_forward_marginals(ptr(scores), ptr(lengths), B, L1, L2, gap, T,
                                         *[ptr(o) for o in outs], ptr(ws), nbytes, stream()))
    _check_status(ws, B)
    return tuple(outs)


def swa_forward_marginals(scores, lengths, go, ge, T, fam="swa"):
    """Affine gap: (partition, marginals, grad_open, grad_ext, grad_T) through the C ABI
    (fam "nwa": global alignment, the value instead of the partition)."""
    import torch
    B, L1, L2 = scores.shape
    dev = scores.device
    lengths = _lengths(lengths, B, L1, L2, dev)
    outs = [torch.empty(B, device=dev), torch.empty(B, L1, L2, device=dev)] + \
        [torch.empty(B, device=dev) for _ in range(3)]
    nbytes = getattr(lib(), f"d2p_{fam}_workspace_bytes")(B, L1, L2)
    ws = _workspace(nbytes, dev)
    check(getattr(lib(), f"d2p_{fam}_forward_marginals")(ptr(scores), ptr(lengths), B, L1, L2,
                                                          go, ge, T, *[ptr(o) for o in outs],
                                                          ptr(ws), nbytes, stream()))
    _check_status(ws, B)
    return tuple(outs)


def dtw_forward_marginals(costs, lengths, T, bandwidth=-1):
    """Soft DTW: (value, marginals, grad_T) through the C ABI."""
    import torch
    B, L1, L2 = costs.shape
    dev = costs.device
    lengths = _lengths(lengths, B, L1, L2, dev)
    outs = [torch.empty(B, device=dev), torch.empty(B, L1, L2, device=dev),
            torch.empty(B, device=dev)]
    nbytes = lib().d2p_dtw_workspace_bytes(B, L1, L2)
    ws = _workspace(nbytes, dev)
    check(lib().d2p_dtw_forward_marginals(ptr(costs), ptr(lengths), B, L1, L2, T, bandwidth,
                                          *[ptr(o) for o in outs], ptr(ws), nbytes, stream()))
    _check_status(ws, B)
    return tuple(outs)


def _second_ws(B, L1, L2, dev, fam="sw"):
    nbytes = getattr(lib(), f"d2p_{fam}_second_workspace_bytes")(B, L1, L2)
    return _workspace(nbytes, dev), nbytes


def sw_hvp(scores, V, lengths, gap, T, fam="sw"):
    import torch
    B, L1, L2 = scores.shape
    dev = scores.device
    lengths = _lengths(lengths, B, L1, L2, dev)
    out = torch.empty(B, L1, L2, device=dev)
    ws, nbytes = _second_ws(B, L1, L2, dev, fam)
    check(getattr(lib(), f"d2p_{fam}_hvp")(ptr(scores), ptr(V), ptr(lengths), B, L1, L2, gap,
                                            T, ptr(out), ptr(ws), nbytes, stream()))
    _check_status(ws, B)
    return out


def sw_param_jacobian(scores, ptype, lengths, gap, T, fam="sw"):
    import torch
    B, L1, L2 = scores.shape
    dev = scores.device
    lengths = _lengths(lengths, B, L1, L2, dev)
    out = torch.empty(B, L1, L2, device=dev)
    ws, nbytes = _second_ws(B, L1, L2, dev, fam)
    check(getattr(lib(), f"d2p_{fam}_param_jacobian")(ptr(scores), ptype, ptr(lengths), B, L1,
                                                       L2, gap, T, ptr(out), ptr(ws), nbytes,
                                                       stream()))
    _check_status(ws, B)
    return out


def sw_backward_full(scores, grad_alignment, lengths, gap, T, fam="sw"):
    import torch
    B, L1, L2 = scores.shape
    dev = scores.device
    lengths = _lengths(lengths, B, L1, L2, dev)
    gs = torch.empty(B, L1, L2, device=dev)
    gg = torch.empty(B, device=dev)
    gt = torch.empty(B, device=dev)
    ws, nbytes = _second_ws(B, L1, L2, dev, fam)
    check(getattr(lib(), f"d2p_{fam}_backward_full")(ptr(scores), ptr(grad_alignment),
                                                      ptr(lengths), B, L1, L2, gap, T, ptr(gs),
                                                      ptr(gg), ptr(gt), ptr(ws), nbytes,
                                                      stream()))
    _check_status(ws, B)
    return gs, gg, gt


def _swa_second_ws(B, L1, L2, dev, fam="swa"):
    nbytes = getattr(lib(), f"d2p_{fam}_second_workspace_bytes")(B, L1, L2)
    return _workspace(nbytes, dev), nbytes


def swa_hvp(scores, V, lengths, go, ge, T, fam="swa"):
    import torch
    B, L1, L2 = scores.shape
    dev = scores.device
    lengths = _lengths(lengths, B, L1, L2, dev)
    out = torch.empty(B, L1, L2, device=dev)
    ws, nbytes = _swa_second_ws(B, L1, L2, dev, fam)
    check(getattr(lib(), f"d2p_{fam}_hvp")(ptr(scores), ptr(V), ptr(lengths), B, L1, L2, go, ge,
                                           T, ptr(out), ptr(ws), nbytes, stream()))
    _check_status(ws, B)
    return out


def swa_param_jacobian(scores, ptype, lengths, go, ge, T, fam="swa"):
    import torch
    B, L1, L2 = scores.shape
    dev = scores.device
    lengths = _lengths(lengths, B, L1, L2, dev)
    out = torch.empty(B, L1, L2, device=dev)
    ws, nbytes = _swa_second_ws(B, L1, L2, dev, fam)
    check(getattr(lib(), f"d2p_{fam}_param_jacobian")(ptr(scores), ptype, ptr(lengths), B, L1,
                                                      L2, go, ge, T, ptr(out), ptr(ws), nbytes,
                                                      stream()))
    _check_status(ws, B)
    return out


def swa_backward_full(scores, grad_alignment, lengths, go, ge, T, fam="swa"):
    import torch
    B, L1, L2 = scores.shape
    dev = scores.device
    lengths = _lengths(lengths, B, L1, L2, dev)
    gs = torch.empty(B, L1, L2, device=dev)
    gp = [torch.empty(B, device=dev) for _ in range(3)]
    ws, nbytes = _swa_second_ws(B, L1, L2, dev, fam)
    check(getattr(lib(), f"d2p_{fam}_backward_full")(ptr(scores), ptr(grad_alignment),
                                                     ptr(lengths), B, L1, L2, go, ge, T, ptr(gs),
                                                     *[ptr(g) for g in gp], ptr(ws), nbytes,
                                                     stream()))
    _check_status(ws, B)
    return (gs, *gp)


def nwa_forward_marginals(scores, lengths, go, ge, T):
    """Affine-gap NW: (value, marginals, grad_open, grad_ext, grad_T) through the C ABI."""
    return swa_forward_marginals(scores, lengths, go, ge, T, fam="nwa")


def nwa_hvp(scores, V, lengths, go, ge, T):
    return swa_hvp(scores, V, lengths, go, ge, T, fam="nwa")


def nwa_param_jacobian(scores, ptype, lengths, go, ge, T):
    return swa_param_jacobian(scores, ptype, lengths, go, ge, T, fam="nwa")


def nwa_backward_full(scores, grad_alignment, lengths, go, ge, T):
    return swa_backward_full(scores, grad_alignment, lengths, go, ge, T, fam="nwa")


def dtw_hvp(costs, V, lengths, T, bw=-1):
    import torch
    B, L1, L2 = costs.shape
    dev = costs.device
    lengths = _lengths(lengths, B, L1, L2, dev)
    out = torch.empty(B, L1, L2, device=dev)
    nbytes = lib().d2p_dtw_second_workspace_bytes(B, L1, L2)
    ws = _workspace(nbytes, dev)
    check(lib().d2p_dtw_hvp(ptr(costs), ptr(V), ptr(lengths), B, L1, L2, T, bw, ptr(out),
                            ptr(ws), nbytes, stream()))
    _check_status(ws, B)
    return out


def dtw_param_jacobian(costs, lengths, T, bw=-1):
    import torch
    B, L1, L2 = costs.shape
    dev = costs.device
    lengths = _lengths(lengths, B, L1, L2, dev)
    out = torch.empty(B, L1, L2, device=dev)
    nbytes = lib().d2p_dtw_second_workspace_bytes(B, L1, L2)
    ws = _workspace(nbytes, dev)
    check(lib().d2p_dtw_param_jacobian(ptr(costs), ptr(lengths), B, L1, L2, T, bw, ptr(out),
                                       ptr(ws), nbytes, stream()))
    _check_status(ws, B)
    return out


def dtw_backward_full(costs, ga, lengths, T, bw=-1):
    import torch
    B, L1, L2 = costs.shape
    dev = costs.device
    lengths = _lengths(lengths, B, L1, L2, dev)
    gc = torch.empty(B, L1, L2, device=dev)
    gt = torch.empty(B, device=dev)
    nbytes = lib().d2p_dtw_second_workspace_bytes(B, L1, L2)
    ws = _workspace(nbytes, dev)
    check(lib().d2p_dtw_backward_full(ptr(costs), ptr(ga), ptr(lengths), B, L1, L2, T, bw,
                                      ptr(gc), ptr(gt), ptr(ws), nbytes, stream()))
    _check_status(ws, B)
    return gc, gt


def scale_by_batch(src, g):
    import torch
    out = torch.empty_like(src)
    B = src.shape[0]
    check(lib().d2p_scale_by_batch(ptr(src), ptr(g), ptr(out), B, src.numel() // B, stream()))
    return out


def scale_by_batch_strided(src, g):
    """g: a 1-d view with one factor per batch row, any non-negative stride."""
    import torch
    out = torch.empty_like(src)
    B = src.shape[0]
    check(lib().d2p_scale_by_batch_strided(ptr(src), ptr(g), g.stride(0), ptr(out), B,
                                           src.numel() // B, stream()))
    return out


def scale_by_batch_lengths(src, g, lengths):
    """src [B, L1, L2] zero outside lengths (int32 [B, 2] on the device, or None)."""
    import torch
    out = torch.empty_like(src)
    B, L1, L2 = src.shape
    check(lib().d2p_scale_by_batch_lengths(ptr(src), ptr(g), g.stride(0),
                                           ptr(lengths) if lengths is not None else None,
                                           ptr(out), B, L1, L2, stream()))
    return out


def nw_hvp(scores, V, lengths, gap, T):
    return sw_hvp(scores, V, lengths, gap, T, fam="nw")


def nw_param_jacobian(scores, ptype, lengths, gap, T):
    return sw_param_jacobian(scores, ptype, lengths, gap, T, fam="nw")


def nw_backward_full(scores, grad_alignment, lengths, gap, T):
    return sw_backward_full(scores, grad_alignment, lengths, gap, T, fam="nw")


def dtw_sqeuclid_forward_marginals(x, y, lengths, T, bandwidth=-1):
    """Fused squared-Euclidean soft DTW: (value, marginals, grad_T) through the C ABI."""
    import torch
    B, L1, D = x.shape
    L2 = y.shape[1]
    dev = x.device
    lengths = _lengths(lengths, B, L1, L2, dev)
    outs = [torch.empty(B, device=dev), torch.empty(B, L1, L2, device=dev),
            torch.empty(B, device=dev)]
    nbytes = lib().d2p_dtw_workspace_bytes_banded(B, L1, L2, bandwidth)
    ws = _workspace(nbytes, dev)
    check(lib().d2p_dtw_sqeuclid_forward_marginals(ptr(x), ptr(y), ptr(lengths), B, L1, L2, D, T,
                                                   bandwidth, *[ptr(o) for o in outs], ptr(ws),
                                                   nbytes, stream()))
    _check_status(ws, B)
    return tuple(outs)


def sqeuclid_feature_grad(G, x, y, scale=None):
    import torch
    B, L1, D = x.shape
    L2 = y.shape[1]
    gx = torch.empty_like(x)
    gy = torch.empty_like(y)
    check(lib().d2p_sqeuclid_feature_grad(ptr(G), ptr(x), ptr(y),
                                          ptr(scale) if scale is not None else None, B, L1,
                                          L2, D, ptr(gx), ptr(gy), stream()))
    return gx, gy


def pairwise_sqdist(x, y):
    import torch
    B, L1, D = x.shape
    L2 = y.shape[1]
    out = torch.empty(B, L1, L2, device=x.device)
    check(lib().d2p_pairwise_sqdist(ptr(x), ptr(y), B, L1, L2, D, ptr(out), stream()))
    return out

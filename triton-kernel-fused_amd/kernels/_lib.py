"""ctypes binding of libmoe_gfx950.so (the C ABI declared in include/moe_gfx950.h).

Only plain pointers, integers and the HIP stream handle cross this boundary; PyTorch owns every
buffer. A missing library is an error, never a fallback: the MoE entry points have no other
implementation.
"""
import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("MOE_GFX950_LIB",
                          os.path.join(os.path.dirname(_HERE), "libmoe_gfx950.so"))

MOE_DT = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
_S = ctypes.c_size_t
_F = ctypes.c_float

# name -> argtypes (every entry point returns int status unless listed in _RESTYPES)
_SIGS = {
    "moe_version": [],
    "moe_tile_rows": [],
    "moe_get_workspace_size": [_L, _I, _I],
    "moe_token_split_workspace_size": [],
    "moe_dispatch": [_P, _L, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _S, _P],
    "moe_dispatch_noalloc": [_P, _L, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P],
    "moe_grouped_gateup_swiglu_fwd": [_I, _P, _L, _L, _P, _I, _L, _P, _P, _P, _P, _L, _P, _P, _P,
                                      _P, _P],
    "moe_grouped_down_fwd": [_I, _P, _P, _I, _L, _L, _P, _P, _L, _P, _P, _S, _P],
    "moe_combine_fwd": [_I, _P, _P, _P, _P, _P, _I, _I, _P, _L, _I, _L, _I, _P, _P],
    "moe_combine_bwd": [_I, _P, _L, _P, _P, _P, _P, _P, _I, _I, _P, _P, _L, _I, _L, _P, _P, _P],
    "moe_grouped_down_dx_swiglu_bwd": [_I, _P, _P, _I, _L, _L, _P, _P, _P, _P, _L, _P, _P, _P],
    "moe_grouped_down_dx_gated_bwd": [_I, _P, _L, _P, _I, _L, _L, _P, _P, _P, _P, _P, _P, _L,
                                      _P, _P, _P, _P],
    "moe_gate_grad_parts": [_L],
    "moe_gate_grad": [_I, _P, _I, _L, _P, _L, _P, _P, _P, _I, _I, _P, _L, _I, _L, _P, _P],
    "moe_grouped_gateup_dx": [_I, _P, _P, _I, _L, _L, _P, _P, _L, _P, _P, _S, _P],
    "moe_grouped_wgrad": [_I, _P, _L, _P, _P, _L, _P, _L, _L, _P, _P, _I, _I, _P, _P, _S, _P],
    "moe_unpermute_bwd": [_I, _P, _P, _L, _P, _P, _P, _I, _I, _P, _L, _I, _L, _P, _P],
    "moe_glu_fwd": [_I, _P, _L, _P, _P, _P, _I, _L, _L, _P, _L, _P],
    "moe_glu_bwd": [_I, _P, _L, _L, _P, _L, _P, _P, _P, _I, _L, _L, _P, _L, _P, _P, _P],
    "moe_fp8_fwd": [_P, _P, _L, _L, _P, _P, _P, _P, _I, _L, _P, _P, _L, _P, _P, _P, _P],
    "moe_fp8_inter_bscale_bytes": [_L, _L, _I],
    "moe_rowquant_fp8": [_P, _L, _L, _P, _P, _P],
    "moe_router_topk_fwd": [_I, _P, _L, _L, _I, _P, _I, _I, _I, _F, _P, _P, _P, _P],
    "moe_router_topk_bwd": [_I, _P, _L, _L, _I, _P, _P, _I, _I, _I, _F, _P, _L, _P],
    "moe_router_bias_update": [_P, _P, _I, _F, _P],
    "moe_mxfp8_fwd": [_P, _L, _L, _P, _P, _P, _P, _I, _L, _P, _P, _L, _P, _P, _P],
}
_RESTYPES = {"moe_version": ctypes.c_char_p, "moe_gate_grad_parts": ctypes.c_int, "moe_get_workspace_size": ctypes.c_size_t,
             "moe_token_split_workspace_size": ctypes.c_size_t,
             "moe_fp8_inter_bscale_bytes": ctypes.c_int64}

_ERRORS = {
    1: (ValueError, "shape"),
    2: (ValueError, "alignment (16-byte pointers; H and I multiples of 8)"),
    3: (ValueError, "unsupported activation code"),
    4: (TypeError, "dtype"),
    5: (RuntimeError, "HIP launch failure"),
    6: (ValueError, "workspace"),
}

_lib = None
_timer = None   # list collecting (name, start_event, end_event) while a bench times kernels


def set_timer(records):
    """Record a HIP event pair around every entry-point call into `records` (a list), on the
    stream the library launches on (torch's current stream); None switches it off."""
    global _timer
    _timer = records


def declared_symbols():
    return sorted(_SIGS)


def lib():
    """Load the library once; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python triton-kernel-fused_amd/build_lib.py` "
                "(or __graft_entry__.build()); the MoE entry points have no fallback path")
        h = ctypes.CDLL(LIB_PATH)
        for name, argtypes in _SIGS.items():
            fn = getattr(h, name)
            fn.argtypes = argtypes
            fn.restype = _RESTYPES.get(name, ctypes.c_int)
        _lib = h
    return _lib


def call(name, *args, tag=None):
    """Call an int-status entry point and raise the mapped Python exception on failure. `tag`
    only labels the call in timer records (e.g. which weight a wgrad is for)."""
    if _timer is None:
        rc = getattr(lib(), name)(*args)
    else:
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record()
        rc = getattr(lib(), name)(*args)
        ev1.record()
        _timer.append((name if tag is None else f"{name}:{tag}", ev0, ev1))
    if rc != 0:
        exc, what = _ERRORS.get(rc, (RuntimeError, "unknown"))
        raise exc(f"{name} failed: {what} (status {rc})")


def ptr(t):
    """Device pointer of a tensor (None -> NULL)."""
    return None if t is None else t.data_ptr()


_SPLIT_WS = {}
_SPLIT_WS_MAX = 4   # workspaces kept (one per (device, stream)); older ones are dropped


def split_workspace(device):
    """The token GEMMs' split workspace for `device` and its current stream: zero-filled once and
    kept zero by the kernels; one per stream, since calls that share one must be stream-ordered.
    At most _SPLIT_WS_MAX are kept (least recently used dropped), so code that makes a new stream
    per iteration does not accumulate them; a dropped workspace is freed through the caching
    allocator, which orders its reuse after the work already queued on that stream.
    Returns (pointer, bytes)."""
    dev = torch.device(device)
    if dev.index is None:
        dev = torch.device("cuda", torch.cuda.current_device())
    key = (dev.index, stream_of(dev))
    ws = _SPLIT_WS.pop(key, None)
    if ws is None:
        with torch.cuda.device(dev):
            n = lib().moe_token_split_workspace_size()
        if n == 0:
            return None, 0
        ws = torch.zeros(n, device=dev, dtype=torch.uint8)
    _SPLIT_WS[key] = ws                      # most recently used last
    while len(_SPLIT_WS) > _SPLIT_WS_MAX:
        del _SPLIT_WS[next(iter(_SPLIT_WS))]
    return ws.data_ptr(), ws.numel()


def stream_of(device):
    return torch.cuda.current_stream(device).cuda_stream


def dtype_code(dt):
    try:
        return MOE_DT[dt]
    except KeyError:
        raise TypeError(f"unsupported dtype {dt}; expected float32, float16 or bfloat16") from None

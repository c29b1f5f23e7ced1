"""ctypes binding of libmi355moe.so (the C ABI declared in include/mi355moe.h).

There is no fallback: if the HIP library is missing or fails to load, every entry point raises. PyTorch is
used only for device memory and streams; tensors are passed as raw device pointers.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmi355moe.so")
CSRC = os.path.join(os.path.dirname(_HERE), "csrc")

_LIB = None

vp = ctypes.c_void_p
i32 = ctypes.c_int
i64 = ctypes.c_int64
u64 = ctypes.c_uint64
f32 = ctypes.c_float
sz = ctypes.c_size_t


class MMLayer(ctypes.Structure):
    """Mirror of mm_layer_t."""

    _fields_ = [("gate_ptr", vp), ("up_ptr", vp), ("down_ptr", vp), ("suh13", vp), ("svh13", vp), ("suh2", vp),
                ("svh2", vp), ("E", i32), ("H", i32), ("I", i32), ("limit", f32), ("flags", i32)]

    EXACT = 1     # MM_LAYER_EXACT: fp16-rounded weights (the reference's EXACT expert) instead of AFFINE


# name -> (restype, argtypes)
_SIGS = {
    "mm_version": (i32, []),
    "mm_last_error": (ctypes.c_char_p, []),
    "mm_host_alloc": (i32, [ctypes.POINTER(vp), sz]),
    "mm_host_free": (i32, [vp]),
    "mm_router_topk": (i32, [vp, i32, i32, vp, i32, i32, vp, vp, vp, vp]),
    "mm_split": (i32, [vp, vp, vp, i32, i32, i32, i32, vp, vp, vp, vp, vp, vp, vp, i32, vp, vp, vp, vp, vp, vp, vp, vp, vp]),
    "mm_combine_host": (i32, [vp, i32, vp, vp, vp, vp, i64, vp]),
    "mm_permute_workspace": (sz, [i32, i32]),
    "mm_permute": (i32, [vp, vp, i32, i32, i32, vp, vp, vp, vp, vp, vp, vp, vp, vp, sz, vp]),
    "mm_combine": (i32, [vp, vp, vp, vp, i32, i32, i32, i32, i32, vp]),
    "mm_gemv_workspace": (sz, [i32, i32, i32, i32]),
    "mm_expert_gemv": (i32, [ctypes.POINTER(MMLayer), vp, i32, i32, i32, i32, i32, vp, vp, vp, vp, vp, i32, vp, vp, sz,
                             i32, vp]),
    "mm_moe_decode": (i32, [ctypes.POINTER(MMLayer), vp, i32, i32, i32, i32, vp, vp, i32, vp, vp, sz, vp]),
    "mm_moe_decode_noalloc": (i32, [ctypes.POINTER(MMLayer), vp, i32, i32, i32, i32, vp, vp, i32, vp, vp]),
    "mm_prefill_workspace": (sz, [i32, i32, i32, i32]),
    "mm_grouped_gemm": (i32, [ctypes.POINTER(MMLayer), vp, i32, i32, i32, vp, i32, vp, vp, sz, vp]),
    "mm_moe_prefill": (i32, [ctypes.POINTER(MMLayer), vp, i32, i32, i32, vp, vp, i32, i32, vp, vp, sz, vp]),
    "mm_fused_moe_workspace": (sz, [i32, i32, i32, i32, i32, i32]),
    "mm_fused_moe": (i32, [ctypes.POINTER(MMLayer), vp, i32, i32, i32, vp, vp, i32, vp, vp, sz, vp]),
    "mm_fat_batched_workspace": (sz, [i32, i32, i32, i32, i32]),
    "mm_fat_batched": (i32, [ctypes.POINTER(MMLayer), vp, i32, i32, i32, vp, vp, vp, vp, i32, vp, vp, sz, vp]),
    "mm_slot_point": (i32, [vp, vp, vp, vp, i32, vp, i32, vp]),
    "mm_stage_copy": (i32, [vp, vp, vp, i32, vp]),
    "mm_copy_stream": (i32, [i32, i32, vp, ctypes.POINTER(vp)]),
    "mm_read_probe": (i32, [vp, u64, vp, i32, vp]),
    "mm_synth_u16": (i32, [vp, u64, u64, u64, vp]),
    "mm_synth_layer": (i32, [ctypes.POINTER(MMLayer), u64, vp]),
    "mm_expert_seed": (u64, [u64, u64]),
    "mm_prepare_input": (i32, [vp, i32, i32, i32, vp, vp, vp]),
    "mm_tier_init": (i32, [i32, vp, i32, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32]),
    "mm_tier_add_layer": (i32, [i32, i32, vp, vp, vp, vp, vp, vp, vp]),
    "mm_tier_set_limit": (i32, [f32]),
    "mm_tier_set_mode": (i32, [i32]),
    "mm_tier_start": (i32, [i32]),
    "mm_tier_stop": (i32, []),
    "mm_tier_shutdown": (i32, []),
    "mm_tier_forward": (i32, [i32, vp, i32, vp, vp, i32, vp, i32]),
    "mm_tier_stats": (i32, [vp]),
}

EXPORTS = tuple(_SIGS)

# element types of a layer input (MM_DTYPE_* in include/mi355moe.h)
DTYPE_F16, DTYPE_BF16, DTYPE_F32 = 0, 1, 2


def load():
    """Load the library (raises if it is absent: the HIP path is the only path)."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"mi355moe: HIP library not built ({LIB_PATH} missing); run __graft_entry__.build()")
    L = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in _SIGS.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = L
    return L


def check(rc, what=""):
    if rc != 0:
        msg = load().mm_last_error().decode(errors="replace")
        raise RuntimeError(f"mi355moe {what}: error {rc}: {msg}")
    return rc


def call(name, *args):
    return check(getattr(load(), name)(*args), name)


def call_count(name, *args):
    """Entry points that return a count (>= 0) or a negative error."""
    rc = getattr(load(), name)(*args)
    if rc < 0:
        check(rc, name)
    return rc


def ptr(t):
    """Device (or host) address of a tensor, or None for NULL."""
    if t is None:
        return None
    return t.data_ptr()


def stream_ptr(stream=None):
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


# copy stream roles (index of mm_copy_stream)
COPY_STAGING, COPY_CACHE = 0, 1
COPY_UNVERIFIED = 1
_COPY_STREAMS = {}


def copy_stream(device, index, compute=None):
    """torch stream over the library's copy stream `index` of `device` for work that overlaps `compute` (default:
    the device's current stream): a stream checked to run on another hardware queue than `compute`."""
    import warnings
    import torch
    dev = torch.device(device)
    d = dev.index if dev.index is not None else torch.cuda.current_device()
    comp = compute if compute is not None else torch.cuda.current_stream(d)
    key = (d, index, comp.cuda_stream)
    s = _COPY_STREAMS.get(key)
    if s is None:
        out = vp()
        rc = load().mm_copy_stream(d, index, comp.cuda_stream, ctypes.byref(out))
        if rc == COPY_UNVERIFIED:
            warnings.warn(f"mi355moe: no copy stream on device {d} was seen to run beside the compute stream; copies "
                          "may serialise with compute (raise GPU_MAX_HW_QUEUES)")
        elif rc != 0:
            check(rc, "mm_copy_stream")
        s = _COPY_STREAMS[key] = torch.cuda.ExternalStream(out.value, device=torch.device("cuda", d))
    return s

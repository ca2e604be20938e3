"""ctypes binding of libsmel_moe.so (the C-ABI declared in include/smel_moe.h, smel_f32.h, smel_norm.h, smel_stream.h and
smel_loss.h).

The library is the only compute path: if it is missing, or no GPU is visible, calls raise instead of falling back to
anything else. Tensors go in as raw device pointers; every call runs on torch's current HIP stream.
"""
from __future__ import annotations

import ctypes
import os

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
# SMEL_MOE_LIB names another build of the same library (e.g. one compiled with different flags)
LIB_PATH = os.environ.get("SMEL_MOE_LIB") or os.path.join(HERE, "libsmel_moe.so")

KIND_INT4, KIND_BF16, KIND_SEL, KIND_SHARED = 0, 1, 2, 3
PACK_Q4, PACK_SZ, PACK_BF16 = 0, 1, 2
WSET_FAST_DQ = 1     # smel_wset.flags: the int4 bank passed smel_int4_fast_ok
WSET_EXT2 = 2        # smel_wset.flags: the LoRA K-extension of the gate_up projection has two 32-wide planes
WSET_XCD_CHUNK = 4   # smel_wset.flags: group-ordered tile list, a contiguous chunk of it per XCD
WSET_MERGE_SHORT = 8 # smel_wset.flags: gate_up forward, a full int4 tile also takes the group's short last tile
WSET_MERGED_LIST = 16 # smel_wset.flags: gate_up forward on smel_dispatch's merged tile list (int4 tiles up to 160 rows)
ABI_VERSION = 23

vp, i64, i32, f32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_float


class WSet(ctypes.Structure):
    """smel_wset of include/smel_moe.h."""
    _fields_ = [("q4", vp), ("sz4", vp), ("wb", vp), ("wsel", vp), ("wsh", vp), ("ext_sel", vp), ("ext_sh", vp),
                ("R", i64), ("C", i64), ("group", i32), ("flags", i32)]


class WSetF32(ctypes.Structure):
    """smel_wset_f32 of include/smel_f32.h."""
    _fields_ = [("q4", vp), ("scale", vp), ("zero", vp), ("wf", vp), ("wsel", vp), ("wsh", vp), ("R", i64), ("C", i64),
                ("group", i32), ("kinds", i32), ("q4_round_bf16", i32), ("pad_", i32)]


class WgDest(ctypes.Structure):
    """smel_wg_dest of include/smel_moe.h."""
    _fields_ = [("ptr", vp), ("s_idx", i64), ("s_p", i64), ("s_q", i64), ("p0", i32), ("np", i32), ("q0", i32),
                ("nq", i32)]


class WgJob(ctypes.Structure):
    """smel_wg_job of include/smel_moe.h."""
    _fields_ = [("L", vp), ("Rm", vp), ("ldr", i64), ("r_rows", i64), ("r_gather", i32), ("use_w", i32), ("Q", i64),
                ("ldl", i64), ("dest", (WgDest * 2) * 2)]


class FwdLoraRows(ctypes.Structure):
    """smel_fwd_lora_rows of include/smel_moe.h: the down LoRA's rows produced in the gate_up forward's epilogue."""
    _fields_ = [("a_sel", vp), ("a_sh", vp), ("scale_sel", ctypes.c_float), ("scale_sh", ctypes.c_float),
                ("part", vp), ("parts", i32), ("ext_out", vp)]


class BwdLoraRows(ctypes.Structure):
    """smel_bwd_lora_rows of include/smel_moe.h: the gate_up LoRA's backward rows produced in the down backward's
    epilogue."""
    _fields_ = [("bt_sel", vp), ("bt_sh", vp), ("scale_sel", ctypes.c_float), ("scale_sh", ctypes.c_float),
                ("n_sel", i32), ("planes", i32), ("part", vp), ("parts", i32)]


class LoraSet(ctypes.Structure):
    """smel_lora_set of include/smel_moe.h: one LoRA set's fp32 factors and its bf16 layouts."""
    _fields_ = [(n, vp) for n in ("A_gate", "B_gate", "A_up", "B_up", "A_down", "B_down")] + \
               [("n", i64), ("r", i64)] + \
               [(n, vp) for n in ("fwd_gu", "fwd_dn", "a_gu", "a_dn", "bt_dn", "bt_gu", "at_gu", "at_dn")]


class H2DRegion(ctypes.Structure):
    """smel_h2d_region of include/smel_stream.h."""
    _fields_ = [("dst", vp), ("src", vp), ("bytes", i64)]


# name -> (restype, argtypes)
SIGNATURES = {
    "smel_last_error": (ctypes.c_char_p, []),
    "smel_abi_version": (i32, []),
    "smel_dequant_int4": (i32, [vp, vp, vp, vp, i64, i64, i64, i32, vp]),
    "smel_quantize_int4": (i32, [vp, i32, i64, i64, i32, ctypes.POINTER(f32), i32, vp, vp, vp, vp]),
    "smel_packed_bytes": (i64, [i32, i64, i64]),
    "smel_pack_int4": (i32, [vp, vp, vp, i64, i64, i64, vp, vp, vp]),
    "smel_pack_bf16": (i32, [vp, i64, i64, i64, vp, vp]),
    "smel_packed_t_bytes": (i64, [i32, i64, i64, i64, i64]),
    "smel_pack_int4_t": (i32, [vp, vp, vp, i64, i64, i64, i64, i32, vp, vp, vp]),
    "smel_int4_fast_ok": (i32, [vp, vp, i64, vp, vp]),
    "smel_pack_bf16_t": (i32, [vp, i64, i64, i64, i64, vp, vp]),
    "smel_route": (i32, [vp, vp, vp, i64, i64, i64, i64, vp, vp, vp, vp, vp, vp, vp, vp]),
    "smel_route_counted": (i32, [vp, vp, vp, i64, i64, i64, i64, vp, vp, vp, vp, vp, vp, vp, vp, vp]),
    "smel_route_ld": (i64, [i64, i32]),
    "smel_route_logits": (i32, [vp, i64, i64, i64, vp, vp, vp, vp, vp]),
    "smel_dispatch": (i32, [vp, i32, i64, i64, i64, i64, i32, vp, vp, vp, vp, vp, vp, vp, vp, vp, i32, vp, vp, vp, vp]),
    "smel_dispatch_counted": (i32, [vp, i32, i64, i64, i64, i64, i32, vp, vp, vp, vp, vp, vp, vp, vp, vp, i32, vp, vp, vp,
                                    vp]),
    "smel_dispatch_ws_size": (i64, [i64, i64]),
    "smel_dispatch_max_tiles": (i64, [i64, i64, i64, i32]),
    "smel_dispatch_noalloc": (i32, [vp, i32, i64, i64, i64, i64, i32, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp]),
    "smel_dispatch_noalloc_max_ws": (i64, []),
    "smel_lora_prep": (i32, [vp, vp, vp, vp, vp, vp, i64, i64, i32, i64, i64, vp, vp, vp, vp, vp, vp, vp, vp, vp]),
    "smel_lora_prep_sets": (i32, [ctypes.POINTER(LoraSet), i32, i32, i64, i64, vp]),
    "smel_lora_ext": (i32, [vp, vp, i64, vp, vp, i64, i64, i32, vp, i64, i64, vp, vp, i64, f32, f32, vp, i64, vp]),
    "smel_gmm_fwd": (i32, [ctypes.POINTER(WSet), vp, vp, vp, i64, vp, i64, i64, i32, vp, i64, i64, vp, i32, i32,
                           vp, i64, vp, vp]),
    "smel_gmm_fwd_lr": (i32, [ctypes.POINTER(WSet), vp, vp, vp, i64, vp, i64, i64, i32, vp, i64, i64, vp, i32, i32,
                              vp, i64, vp, ctypes.POINTER(FwdLoraRows), vp]),
    "smel_gmm_fwd_nblocks": (i64, [i64, i32]),
    "smel_combine": (i32, [vp, vp, vp, vp, vp, i64, i64, i64, vp, vp]),
    "smel_gmm_bwd": (i32, [ctypes.POINTER(WSet), vp, vp, vp, i64, vp, i64, i64, i32, vp, i64, i64, vp, i32, i32,
                           vp, vp, vp, vp, i64, vp, vp]),
    "smel_gmm_bwd_lr": (i32, [ctypes.POINTER(WSet), vp, vp, vp, i64, vp, i64, i64, i32, vp, i64, i64, vp, i32, i32,
                              vp, vp, vp, vp, i64, vp, ctypes.POINTER(BwdLoraRows), vp]),
    "smel_gmm_bwd_nblocks": (i64, [i64]),
    "smel_lora_rows_sum": (i32, [vp, vp, i64, vp, i32, i32, vp, i32, i32, vp, vp]),
    "smel_route_bwd": (i32, [vp, i64, vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, vp, i64, vp, vp, vp]),
    "smel_route_gemma4": (i32, [vp, vp, vp, vp, i64, i64, i64, i64, f32, vp, vp, vp, vp, vp, vp, vp, vp]),
    "smel_route_gemma4_prenorm_bwd": (i32, [vp, vp, vp, vp, i64, i64, vp, vp]),
    "smel_dtopv": (i32, [vp, i64, vp, i64, vp, vp]),
    "smel_dx_reduce": (i32, [vp, vp, vp, i32, vp, i64, i64, i64, vp, vp]),
    "smel_lora_wgrad": (i32, [ctypes.POINTER(WgJob), i32, vp, i64, i64, vp, i64, i64, i64, i64, vp, vp, vp, i64, vp,
                              i64, vp]),
    "smel_lora_wgrad_ws_floats": (i64, [ctypes.POINTER(WgJob), i32, i64, i64]),
    # include/smel_f32.h
    "smel_gmm_f32": (i32, [ctypes.POINTER(WSetF32), i32, vp, vp, vp, i64, vp, i64, f32, f32, vp, i64, vp]),
    "smel_wgrad_f32": (i32, [vp, i64, vp, i64, vp, vp, i32, i64, i64, f32, vp, i64, vp]),
    "smel_gather_rows_f32": (i32, [vp, i64, vp, i32, vp, i64, i64, vp, vp]),
    "smel_act_gate_f32": (i32, [vp, i64, i64, i64, i32, vp, i64, vp]),
    "smel_act_gate_bwd_f32": (i32, [vp, i64, vp, i64, i64, i64, i32, vp, i64, vp]),
    "smel_combine_f32": (i32, [vp, vp, vp, i64, i64, i64, vp, vp]),
    "smel_combine_bwd_f32": (i32, [vp, vp, vp, vp, i64, i64, i64, vp, vp, vp]),
    "smel_dx_reduce_f32": (i32, [vp, vp, i64, i64, i64, vp, vp]),
    "smel_route_select_f32": (i32, [vp, i64, i64, i64, i64, vp, vp, vp, vp, vp, vp]),
    "smel_route_bwd_f32": (i32, [vp, vp, vp, vp, i64, i64, i64, vp, vp]),
    "smel_route_prenorm_f32": (i32, [vp, vp, i64, i64, f32, f32, vp, vp, vp]),
    "smel_route_prenorm_bwd_f32": (i32, [vp, vp, vp, vp, i64, i64, f32, vp, vp]),
    "smel_gate_mul_f32": (i32, [vp, vp, vp, i64, i64, vp, vp]),
    "smel_gate_mul_bwd_f32": (i32, [vp, vp, vp, i64, i64, vp, vp, vp]),
    # include/smel_norm.h
    "smel_rmsnorm_fwd": (i32, [vp, i64, i64, i64, vp, i32, f32, i32, vp, vp, vp]),
    "smel_rmsnorm_bwd": (i32, [vp, vp, i64, i64, i64, vp, i32, vp, vp, i32, vp, vp]),
    "smel_add_rmsnorm_fwd": (i32, [vp, vp, i64, i64, vp, i32, f32, i32, vp, vp, vp, vp]),
    "smel_gated_rmsnorm_fwd": (i32, [vp, vp, i64, i64, vp, f32, i32, vp, vp, vp]),
    "smel_gated_rmsnorm_bwd": (i32, [vp, vp, vp, i64, i64, vp, vp, i32, vp, vp, vp]),
    # include/smel_stream.h
    "smel_event_create": (i32, [ctypes.POINTER(vp)]),
    "smel_event_destroy": (i32, [vp]),
    "smel_event_record": (i32, [vp, vp]),
    "smel_stream_wait": (i32, [vp, vp]),
    "smel_h2d_regions": (i32, [ctypes.POINTER(H2DRegion), i32, i64, ctypes.POINTER(vp), ctypes.POINTER(vp), i32, vp]),
    # include/smel_loss.h
    "smel_ce_begin": (i32, [vp, vp, vp, vp, vp, i64, vp]),
    "smel_ce_logits": (i32, [vp, i64, i64, i64, vp, i64, i64, i64, vp, f32, i32, vp, i64, vp, vp, i64, vp, vp, vp]),
    "smel_ce_stats": (i32, [vp, vp, i64, i64, i64, vp, vp, vp, vp, vp]),
    "smel_ce_grad": (i32, [vp, i64, i64, vp, i64, i64, vp, i64, vp, i64, i32, i32, vp, vp, vp]),
    "smel_ce_finish": (i32, [vp, vp, vp, vp, vp, vp, vp, i64, vp, vp, i64, i64, i64, i32, f32, vp, i64, i32, vp, vp]),
    "smel_ce_loss_sum": (i32, [vp, i64, f32, i32, vp, vp]),
    "smel_ce_scale": (i32, [vp, i64, i32, vp, vp]),
    "smel_ce_transpose": (i32, [vp, i64, i64, i64, vp, i64, i32, vp]),
    # include/smel_probe.h
    "smel_probe_mfma": (i32, [vp, i32, i32, vp]),
    "smel_probe_read": (i32, [vp, i64, vp, i32, vp]),
    "smel_probe_copy": (i32, [vp, vp, i64, i32, vp]),
}

_lib = None


class SmelError(RuntimeError):
    pass


def load(path: str = LIB_PATH):
    """Load (once) and type the C-ABI library. Raises if it is missing: there is no other compute path."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise ImportError(f"{path} is missing: build the HIP extension first (python -c 'import __graft_entry__ as g; "
                          f"g.build()')")
    L = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    if L.smel_abi_version() != ABI_VERSION:
        raise ImportError(f"{path} has ABI version {L.smel_abi_version()}, this binding expects {ABI_VERSION}: "
                          f"rebuild the HIP extension")
    _lib = L
    return L


_timing = None   # list of (tag, start event, end event) while timing is on


def call(name: str, *args, tag: str | None = None):
    """Call an entry point that returns a status code; raise SmelError with the library's message on failure.
    While :func:`timing` is active, the launch is bracketed by events on the current stream."""
    fn = getattr(load(), name)
    if _timing is not None:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        rc = fn(*args)
        e1.record()
        _timing.append((tag or name, e0, e1))
    else:
        rc = fn(*args)
    if rc != 0:
        msg = load().smel_last_error().decode(errors="replace")
        raise SmelError(f"{name} failed ({rc}): {msg}")


class timing:
    """Context manager: time every entry-point call (HIP events on the stream the kernels run on). After a device
    synchronize, ``results()`` returns {tag: [milliseconds per call]}."""

    def __enter__(self):
        global _timing
        _timing = []
        self._rec = _timing
        return self

    def __exit__(self, *exc):
        global _timing
        _timing = None
        return False

    def results(self):
        out = {}
        for tag, e0, e1 in self._rec:
            out.setdefault(tag, []).append(e0.elapsed_time(e1))
        return out


def ptr(t: torch.Tensor | None):
    """Device pointer of a tensor (None -> NULL). The tensor must stay alive for the duration of the launch."""
    if t is None:
        return None
    return t.data_ptr()


def stream():
    return torch.cuda.current_stream().cuda_stream


def require_device(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("smel MoE kernels run on the GPU: every tensor must be on a cuda device")

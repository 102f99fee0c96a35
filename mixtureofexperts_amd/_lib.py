"""ctypes binding of libmoe_mi355x.so (C ABI in include/moe_mi355x.h).

There is no fallback: if the shared library is missing or fails to load, every
call raises.  The library is built in-tree by ``mixtureofexperts_amd.build``
(or ``__graft_entry__.build()``).
"""
import ctypes
import os

from .build import LIB_PATH

MOE_OK = 0
MOE_EINVAL = -1
MOE_EOOM = -2
MOE_EHIP = -3
MOE_ENOTREADY = -4
MOE_EUNSUPPORTED = -5
STATUS_NAMES = {
    MOE_EINVAL: "MOE_EINVAL",
    MOE_EOOM: "MOE_EOOM",
    MOE_EHIP: "MOE_EHIP",
    MOE_ENOTREADY: "MOE_ENOTREADY",
    MOE_EUNSUPPORTED: "MOE_EUNSUPPORTED",
}

MOE_F32, MOE_BF16, MOE_FP8_E4M3 = 0, 1, 2
MOE_LAYOUT_FLUX_OUT_IN, MOE_LAYOUT_LLAMA_IN_OUT = 0, 1
MOE_EXPERT_GATED, MOE_EXPERT_STANDARD = 0, 1
MOE_ACT_GELU, MOE_ACT_SILU, MOE_ACT_RELU, MOE_ACT_IDENTITY = 0, 1, 2, 3
MOE_GATE_TOPK, MOE_GATE_SWITCH, MOE_GATE_SHARED, MOE_GATE_SOFT, MOE_GATE_EXPERT_CHOICE = 0, 1, 2, 3, 4
MOE_INIT_COPY, MOE_INIT_PERTURB, MOE_INIT_SPLIT, MOE_INIT_RANDOM = 0, 1, 2, 3
MOE_MAX_TOPK = 16
MOE_MAX_EXPERTS = 512

# every symbol the header declares (checked by the CPU test suite)
EXPORTED_SYMBOLS = [
    "moe_create", "moe_destroy", "moe_last_error", "moe_abi_version",
    "moe_router_outputs", "moe_slots_per_token", "moe_set_router", "moe_set_router_noise", "moe_set_expert_dropout", "moe_router_lse", "moe_set_expert",
    "moe_compute_gates", "moe_route_from_logits", "moe_forward", "moe_expert_forward",
    "moe_forward_async", "moe_stage_router_async", "moe_stage_permute_async",
    "moe_stage_expert_up_async", "moe_stage_expert_down_async", "moe_stage_combine_async",
    "moe_read_counts", "moe_switch_loss", "moe_z_loss", "moe_decode", "moe_decode_async",
    "moe_set_aux_free", "moe_get_aux_free", "moe_aux_free_update_bias", "moe_forward_routed",
    "moe_init_experts_from_dense", "moe_get_expert", "moe_switch_loss_noalloc",
]


class MoeConfigC(ctypes.Structure):
    _fields_ = [
        ("num_experts", ctypes.c_int32),
        ("expert_type", ctypes.c_int32),
        ("input_dim", ctypes.c_int32),
        ("hidden_dim", ctypes.c_int32),
        ("output_dim", ctypes.c_int32),
        ("activation", ctypes.c_int32),
        ("gate_kind", ctypes.c_int32),
        ("top_k", ctypes.c_int32),
        ("gate_num_shared", ctypes.c_int32),
        ("weight_dtype", ctypes.c_int32),
        ("balance_alpha", ctypes.c_float),
        ("z_loss_weight", ctypes.c_float),
        ("capacity_factor", ctypes.c_float),
        ("drop_tokens", ctypes.c_int32),
        ("max_tokens", ctypes.c_int32),
        ("num_shared_experts", ctypes.c_int32),
        ("gate_param", ctypes.c_float),
        ("reserved", ctypes.c_int32 * 5),
    ]


class MoeForwardAux(ctypes.Structure):
    _fields_ = [
        ("logits", ctypes.c_void_p),
        ("probs", ctypes.c_void_p),
        ("indices", ctypes.c_void_p),
        ("gates", ctypes.c_void_p),
        ("counts", ctypes.c_void_p),
        ("offsets", ctypes.c_void_p),
        ("perm", ctypes.c_void_p),
        ("switch_loss", ctypes.c_void_p),
        ("z_loss", ctypes.c_void_p),
        ("mean_entropy", ctypes.c_void_p),
    ]


class MoeError(RuntimeError):
    def __init__(self, status, message):
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {message}")
        self.status = status


_lib = None


def lib():
    """Load (once) and return the ctypes handle of libmoe_mi355x.so."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python -m mixtureofexperts_amd.build` "
            "(there is no CPU fallback)"
        )
    # One HIP runtime per process.  The torch wheel bundles its own
    # libamdhip64 / libhsa-runtime64 (SONAMEs libamdhip64.so.7 and
    # libhsa-runtime64.so.1) but its own libraries ask for them under other
    # names.  Loading torch first makes this library's dependencies resolve to
    # those already-loaded copies; loading this library first would make torch
    # bring in a second HSA runtime, which then finds no GPU.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    L = ctypes.CDLL(LIB_PATH)
    vp, i32, f32p = ctypes.c_void_p, ctypes.c_int32, ctypes.POINTER(ctypes.c_float)
    L.moe_create.argtypes = [ctypes.POINTER(MoeConfigC), ctypes.POINTER(vp)]
    L.moe_destroy.argtypes = [vp]
    L.moe_last_error.argtypes = [vp]
    L.moe_last_error.restype = ctypes.c_char_p
    L.moe_abi_version.argtypes = []
    L.moe_router_outputs.argtypes = [vp]
    L.moe_slots_per_token.argtypes = [vp]
    L.moe_set_router.argtypes = [vp, vp, vp]
    L.moe_set_router_noise.argtypes = [vp, ctypes.c_float, vp, ctypes.c_uint64]
    L.moe_set_expert_dropout.argtypes = [vp, ctypes.c_float, ctypes.c_uint64]
    L.moe_router_lse.argtypes = [vp, i32, vp]
    L.moe_set_expert.argtypes = [vp, i32, i32, i32, vp, vp, vp, vp, vp, vp, vp, vp]
    L.moe_compute_gates.argtypes = [vp, vp, i32, vp, vp, vp]
    L.moe_route_from_logits.argtypes = [vp, vp, i32, i32, vp, vp, vp, vp, vp, vp]
    L.moe_forward.argtypes = [vp, vp, i32, i32, i32, vp, f32p, ctypes.POINTER(MoeForwardAux)]
    L.moe_forward_routed.argtypes = [vp, vp, i32, i32, i32, vp, vp, i32, vp, vp, f32p, ctypes.POINTER(MoeForwardAux)]
    L.moe_expert_forward.argtypes = [vp, i32, vp, i32, vp]
    L.moe_forward_async.argtypes = [vp, vp, i32, i32, i32, vp, vp, vp]
    L.moe_stage_router_async.argtypes = [vp, vp, i32, i32, i32, vp]
    L.moe_stage_permute_async.argtypes = [vp, vp, i32, i32, vp]
    L.moe_stage_expert_up_async.argtypes = [vp, i32, vp]
    L.moe_stage_expert_down_async.argtypes = [vp, i32, vp]
    L.moe_stage_combine_async.argtypes = [vp, i32, vp, vp]
    L.moe_read_counts.argtypes = [vp, vp]
    L.moe_decode.argtypes = [vp, vp, i32, vp, vp, vp, vp]
    L.moe_decode_async.argtypes = [vp, vp, i32, vp, vp]
    L.moe_switch_loss.argtypes = [vp, i32, i32, vp, i32, ctypes.c_float, f32p]
    L.moe_z_loss.argtypes = [vp, i32, i32, ctypes.c_float, f32p]
    L.moe_switch_loss_noalloc.argtypes = [vp, i32, i32, vp, i32, ctypes.c_float, vp, vp]
    i64, f32 = ctypes.c_int64, ctypes.c_float
    L.moe_set_aux_free.argtypes = [vp, i32, vp, vp, f32, f32, i32, i64, i32, f32]
    L.moe_get_aux_free.argtypes = [vp, vp, vp, ctypes.POINTER(i64)]
    L.moe_aux_free_update_bias.argtypes = [vp, i64, i32, f32, f32, vp, vp]
    L.moe_init_experts_from_dense.argtypes = [vp, i32, i32, vp, vp, vp, vp, vp, vp, i32, f32, ctypes.c_uint64]
    L.moe_get_expert.argtypes = [vp, i32, i32, vp, vp, vp, vp, vp, vp]
    for name in EXPORTED_SYMBOLS:
        if name not in ("moe_last_error",):
            getattr(L, name).restype = ctypes.c_int
    _lib = L
    return L


def check(status, handle=None):
    """Raise MoeError with the library's message for a non-zero status."""
    if status != MOE_OK:
        msg = lib().moe_last_error(handle)
        raise MoeError(status, msg.decode() if msg else "")
    return status

"""Owner of one libmoe_mi355x handle: device-resident weights and workspace.

All array arguments are host numpy arrays in the ABI's token-major memory
order (a Julia (D, T) matrix is passed as its (T, D) row-major memory).
"""
import ctypes
import sys
from collections import namedtuple

import numpy as np

from . import _lib

GateSpec = namedtuple("GateSpec", "kind k num_shared param", defaults=(0.0,))


def _ptr(a):
    return None if a is None else a.ctypes.data


class DeviceLayer:
    def __init__(self, *, num_experts, expert_type, input_dim, hidden_dim, output_dim, activation, gate,
                 weight_dtype, balance_alpha, z_loss_weight, capacity_factor, drop_tokens, max_tokens,
                 num_shared_experts=0):
        c = _lib.MoeConfigC()
        c.num_experts = num_experts
        c.expert_type = expert_type
        c.input_dim = input_dim
        c.hidden_dim = hidden_dim
        c.output_dim = output_dim
        c.activation = activation
        c.gate_kind = gate.kind
        c.top_k = gate.k
        c.gate_num_shared = gate.num_shared
        c.weight_dtype = weight_dtype
        c.balance_alpha = balance_alpha
        c.z_loss_weight = z_loss_weight
        c.capacity_factor = capacity_factor
        c.drop_tokens = int(bool(drop_tokens))
        c.max_tokens = max_tokens
        c.num_shared_experts = int(num_shared_experts)
        c.gate_param = float(gate.param)
        self.cfg = c
        self.max_tokens = max_tokens
        self.num_experts = num_experts
        self.output_dim = output_dim
        self.input_dim = input_dim
        h = ctypes.c_void_p()
        _lib.check(_lib.lib().moe_create(ctypes.byref(c), ctypes.byref(h)), None)
        self.h = h
        self.router_outputs = _lib.lib().moe_router_outputs(h)
        self.slots = _lib.lib().moe_slots_per_token(h)
        # AuxiliaryFreeLoss bias length: the router outputs, or all experts
        # when the layer has shared experts (update_bias! then sees the ids
        # shifted by num_shared_experts, up to num_experts)
        self.aux_free_len = num_experts if num_shared_experts > 0 else self.router_outputs

    @classmethod
    def gating_only(cls, spec, E, T, capacity_factor=None):
        return cls(num_experts=E, expert_type=_lib.MOE_EXPERT_GATED, input_dim=1, hidden_dim=1, output_dim=1,
                   activation=_lib.MOE_ACT_IDENTITY, gate=spec, weight_dtype=_lib.MOE_BF16, balance_alpha=0.0,
                   z_loss_weight=0.0, capacity_factor=1.25 if capacity_factor is None else capacity_factor,
                   drop_tokens=capacity_factor is not None, max_tokens=T)

    def close(self):
        if getattr(self, "h", None) is not None and self.h.value is not None:
            _lib.lib().moe_destroy(self.h)
            self.h = None

    def __del__(self):
        # At interpreter shutdown the HIP runtime, torch's streams and this
        # module's globals may already be torn down: the process is ending,
        # its device memory goes with it, so no device call is made then.
        if sys.is_finalizing():
            return
        try:
            self.close()
        except Exception:
            pass

    # ---- weights --------------------------------------------------------
    def set_router(self, weight_mem_DE, bias=None):
        w = np.ascontiguousarray(weight_mem_DE, dtype=np.float32)
        b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        _lib.check(_lib.lib().moe_set_router(self.h, _ptr(w), _ptr(b)), self.h)

    def set_router_noise(self, noise_scale, noise_weight_mem_DE=None, seed=0):
        """Router noise in training (router.jl:32-41); the noise network's
        weight in the router weight's memory order [D][E_router], or None."""
        w = None if noise_weight_mem_DE is None else np.ascontiguousarray(noise_weight_mem_DE, dtype=np.float32)
        _lib.check(_lib.lib().moe_set_router_noise(self.h, float(noise_scale), _ptr(w), int(seed) & (2**64 - 1)),
                   self.h)

    def router_lse(self, T):
        """Per-token logsumexp of the last routing call's logits (float32 [T])."""
        out = np.zeros(T, np.float32)
        _lib.check(_lib.lib().moe_router_lse(self.h, int(T), out.ctypes.data), self.h)
        return out

    def set_expert_dropout(self, p, seed=0):
        """StandardExpert's Dropout(p) in training (standard.jl:49-51)."""
        _lib.check(_lib.lib().moe_set_expert_dropout(self.h, float(p), int(seed) & (2**64 - 1)), self.h)

    def set_expert(self, e, w1, w2, w3=None, b1=None, b2=None, *, src_dtype=_lib.MOE_F32,
                   layout=_lib.MOE_LAYOUT_LLAMA_IN_OUT, s1=None, s2=None, s3=None):
        """Matrices in memory order of ``layout`` (LLAMA_IN_OUT = [out][in],
        i.e. a numpy (out, in) C-contiguous array)."""
        dt = {_lib.MOE_F32: np.float32, _lib.MOE_BF16: np.uint16, _lib.MOE_FP8_E4M3: np.uint8}[src_dtype]
        conv = lambda a: None if a is None else np.ascontiguousarray(a, dtype=dt)
        convf = lambda a: None if a is None else np.ascontiguousarray(a, dtype=np.float32)
        arrs = [conv(w1), conv(w2), conv(w3), convf(b1), convf(b2), convf(s1), convf(s2), convf(s3)]
        _lib.check(
            _lib.lib().moe_set_expert(self.h, int(e), int(layout), int(src_dtype), *[_ptr(a) for a in arrs]),
            self.h,
        )

    def set_aux_free(self, loss):
        """Load an AuxiliaryFreeLoss's state and parameters into the handle."""
        bias = np.ascontiguousarray(loss.bias, dtype=np.float32)
        mom = np.ascontiguousarray(loss.bias_momentum, dtype=np.float32)
        if bias.size != self.aux_free_len or mom.size != self.aux_free_len:
            raise _lib.MoeError(_lib.MOE_EINVAL, "AuxiliaryFreeLoss.num_experts must equal the router outputs "
                                "(num_experts with shared experts of the layer)")
        _lib.check(_lib.lib().moe_set_aux_free(self.h, 1, bias.ctypes.data, mom.ctypes.data, loss.learning_rate,
                                               loss.momentum, loss.update_freq, loss.update_counter,
                                               int(loss.use_complementary_loss), loss.complementary_weight),
                   self.h)

    def get_aux_free(self, loss):
        """Copy the handle's AuxiliaryFreeLoss state back into ``loss``."""
        bias = np.zeros(self.aux_free_len, dtype=np.float32)
        mom = np.zeros(self.aux_free_len, dtype=np.float32)
        cnt = ctypes.c_int64(0)
        _lib.check(_lib.lib().moe_get_aux_free(self.h, bias.ctypes.data, mom.ctypes.data, ctypes.byref(cnt)),
                   self.h)
        loss.bias, loss.bias_momentum, loss.update_counter = bias, mom, int(cnt.value)

    # ---- calls ------------------------------------------------------------
    def forward(self, x_TD, x_dtype, training, want_aux=False):
        T = x_TD.shape[0]
        out = np.zeros((T, self.output_dim), dtype=np.float32)
        loss = ctypes.c_float(0.0)
        aux, res, keep = self._aux(T, self.slots, want_aux)
        _lib.check(
            _lib.lib().moe_forward(self.h, x_TD.ctypes.data, int(x_dtype), T, int(bool(training)), out.ctypes.data,
                                   ctypes.byref(loss), ctypes.byref(aux)),
            self.h,
        )
        return out, float(np.float32(loss.value)), self._aux_result(res, keep)

    def forward_routed(self, x_TD, x_dtype, training, idx_Tk, gates_Tk, probs_TE=None, want_aux=False):
        """moe_forward_routed: the layer forward on the caller's routing."""
        T = x_TD.shape[0]
        idx = np.ascontiguousarray(idx_Tk, dtype=np.int32)
        gates = np.ascontiguousarray(gates_Tk, dtype=np.float32)
        kd = idx.shape[1]
        probs = None if probs_TE is None else np.ascontiguousarray(probs_TE, dtype=np.float32)
        out = np.zeros((T, self.output_dim), dtype=np.float32)
        loss = ctypes.c_float(0.0)
        aux, res, keep = self._aux(T, kd, want_aux)
        _lib.check(
            _lib.lib().moe_forward_routed(self.h, x_TD.ctypes.data, int(x_dtype), T, int(bool(training)),
                                          idx.ctypes.data, gates.ctypes.data, kd, _ptr(probs), out.ctypes.data,
                                          ctypes.byref(loss), ctypes.byref(aux)),
            self.h,
        )
        return out, float(np.float32(loss.value)), self._aux_result(res, keep)

    def _aux(self, T, slots, want_aux):
        aux = _lib.MoeForwardAux()
        res = {}
        keep = dict(counts=np.zeros(self.num_experts, dtype=np.int32), ent=np.zeros(1, dtype=np.float32),
                    sw=np.zeros(1, dtype=np.float32), zl=np.zeros(1, dtype=np.float32))
        aux.counts = keep["counts"].ctypes.data
        aux.mean_entropy = keep["ent"].ctypes.data
        aux.switch_loss = keep["sw"].ctypes.data
        aux.z_loss = keep["zl"].ctypes.data
        if want_aux:
            res["logits"] = np.zeros((T, self.router_outputs), dtype=np.float32)
            res["probs"] = np.zeros((T, self.router_outputs), dtype=np.float32)
            res["indices"] = np.zeros((T, slots), dtype=np.int32)
            res["gates"] = np.zeros((T, slots), dtype=np.float32)
            res["offsets"] = np.zeros(self.num_experts + 1, dtype=np.int32)
            res["perm"] = np.zeros(T * slots, dtype=np.int32)
            for k in ("logits", "probs", "indices", "gates", "offsets", "perm"):
                setattr(aux, k, res[k].ctypes.data)
        return aux, res, keep

    @staticmethod
    def _aux_result(res, keep):
        res.update(counts=keep["counts"], mean_entropy=float(keep["ent"][0]), switch_loss=float(keep["sw"][0]),
                   z_loss=float(keep["zl"][0]))
        return res

    def expert_forward(self, e, x_nD):
        x = np.ascontiguousarray(x_nD, dtype=np.float32)
        n = x.shape[0]
        y = np.zeros((n, self.output_dim), dtype=np.float32)
        _lib.check(_lib.lib().moe_expert_forward(self.h, int(e), x.ctypes.data, n, y.ctypes.data), self.h)
        return y

    def decode(self, xb_nD):
        """moe_ffn_forward! on n tokens (moe_decode): returns (out [n][Dout],
        logits [n][E], indices [n][k] 1-based, gates [n][k])."""
        x = np.ascontiguousarray(xb_nD, dtype=np.float32)
        n = x.shape[0]
        k = _lib.lib().moe_slots_per_token(self.h)
        out = np.zeros((n, self.output_dim), dtype=np.float32)
        logits = np.zeros((n, self.router_outputs), dtype=np.float32)
        idx = np.zeros((n, k), dtype=np.int32)
        gates = np.zeros((n, k), dtype=np.float32)
        _lib.check(_lib.lib().moe_decode(self.h, x.ctypes.data, n, out.ctypes.data, logits.ctypes.data,
                                         idx.ctypes.data, gates.ctypes.data), self.h)
        return out, logits, idx, gates

"""Expert types of MixtureOfExperts.jl (src/experts/gated.jl,
src/experts/standard.jl).

Weights are held host-side in the reference's Flux shapes, (out, in), and are
uploaded once to the device by the layer that owns them.  Calling an expert
runs its FFN on the device (``moe_expert_forward``).
"""
import numpy as np

from . import _lib
from ._device import DeviceLayer, GateSpec
from .activations import activation_code


class Expert:
    """Abstract expert (src/experts/standard.jl:6)."""

    _dev = None
    _dev_version = -1
    version = 0

    def mark_updated(self):
        """Call after changing weights in place so device copies refresh."""
        self.version += 1

    def _device(self, n):
        if self._dev is None or self._dev_version != self.version or self._dev.max_tokens < n:
            if self._dev is not None:
                self._dev.close()
            dev = DeviceLayer(
                num_experts=1, expert_type=self.expert_type_code, input_dim=self.input_dim,
                hidden_dim=self.hidden_dim, output_dim=self.output_dim,
                activation=activation_code(self.activation), gate=GateSpec(_lib.MOE_GATE_SWITCH, 1, 0),
                weight_dtype=self.weight_dtype, balance_alpha=0.0, z_loss_weight=0.0, capacity_factor=1.0,
                drop_tokens=False, max_tokens=max(n, 128),
            )
            self.upload(dev, 0)
            self._dev, self._dev_version = dev, self.version
        return self._dev

    def __call__(self, x, training=False):
        """(e::Expert)(x; training): x (input_dim, n) -> (output_dim, n)."""
        x = np.asarray(x, dtype=np.float32)
        vec = x.ndim == 1
        xm = x.reshape(-1, 1) if vec else x
        if xm.shape[0] != self.input_dim:
            raise _lib.MoeError(_lib.MOE_EINVAL, f"expert expects input_dim {self.input_dim}, got {xm.shape[0]}")
        n = xm.shape[1]
        y = self._device(n).expert_forward(0, np.ascontiguousarray(xm.T)) if n else np.zeros((0, self.output_dim), np.float32)
        return y[0] if vec else y.T


class GatedExpert(Expert):
    """GatedExpert -- w2(act(w1 x) .* (w3 x)), src/experts/gated.jl:6-35.
    Init: randn * sqrt(2 / input_dim) for all three matrices (:15-27)."""

    expert_type_code = _lib.MOE_EXPERT_GATED

    def __init__(self, input_dim, hidden_dim, output_dim, activation, *, rng=None, weight_dtype=_lib.MOE_F32,
                 w1=None, w2=None, w3=None):
        self.input_dim, self.hidden_dim, self.output_dim = int(input_dim), int(hidden_dim), int(output_dim)
        self.activation = activation
        self.weight_dtype = weight_dtype
        rng = np.random.default_rng() if rng is None else rng
        sigma = np.float32(np.sqrt(np.float32(2.0) / np.float32(input_dim)))
        self.w1 = w1 if w1 is not None else (rng.standard_normal((hidden_dim, input_dim), dtype=np.float32) * sigma)
        self.w2 = w2 if w2 is not None else (rng.standard_normal((output_dim, hidden_dim), dtype=np.float32) * sigma)
        self.w3 = w3 if w3 is not None else (rng.standard_normal((hidden_dim, input_dim), dtype=np.float32) * sigma)
        self.scales = None  # (s1, s2, s3) when w1/w2/w3 hold fp8 e4m3 bytes

    def upload(self, dev, e):
        if self.scales is not None:
            s1, s2, s3 = self.scales
            dev.set_expert(e, self.w1, self.w2, self.w3, src_dtype=_lib.MOE_FP8_E4M3, s1=s1, s2=s2, s3=s3)
        elif self.w1.dtype == np.uint16:
            dev.set_expert(e, self.w1, self.w2, self.w3, src_dtype=_lib.MOE_BF16)
        else:
            dev.set_expert(e, self.w1, self.w2, self.w3, src_dtype=_lib.MOE_F32)


class StandardExpert(Expert):
    """StandardExpert -- w2(act(w1 x .+ b1)) .+ b2, src/experts/standard.jl:8-55.
    Init: w1 randn*sqrt(2/in), w2 randn*sqrt(2/hidden), zero biases (:19-36)."""

    expert_type_code = _lib.MOE_EXPERT_STANDARD

    def __init__(self, input_dim, hidden_dim, output_dim, activation, *, dropout=0.0, bias=True, rng=None,
                 weight_dtype=_lib.MOE_F32, w1=None, w2=None, b1=None, b2=None):
        self.input_dim, self.hidden_dim, self.output_dim = int(input_dim), int(hidden_dim), int(output_dim)
        self.activation = activation
        self.dropout = float(dropout)
        self.weight_dtype = weight_dtype
        rng = np.random.default_rng() if rng is None else rng
        s1 = np.float32(np.sqrt(np.float32(2.0) / np.float32(input_dim)))
        s2 = np.float32(np.sqrt(np.float32(2.0) / np.float32(hidden_dim)))
        self.w1 = w1 if w1 is not None else rng.standard_normal((hidden_dim, input_dim), dtype=np.float32) * s1
        self.w2 = w2 if w2 is not None else rng.standard_normal((output_dim, hidden_dim), dtype=np.float32) * s2
        if bias:
            self.b1 = np.zeros(hidden_dim, np.float32) if b1 is None else np.asarray(b1, np.float32)
            self.b2 = np.zeros(output_dim, np.float32) if b2 is None else np.asarray(b2, np.float32)
        else:
            self.b1 = self.b2 = None
        self.scales = None  # (s1, s2) when w1/w2 hold fp8 e4m3 bytes

    def __call__(self, x, training=False):
        if training and self.dropout > 0:
            raise _lib.MoeError(_lib.MOE_EUNSUPPORTED, "expert dropout in training has no device path")
        return super().__call__(x, training)

    def upload(self, dev, e):
        if self.scales is not None:
            s1, s2 = self.scales
            dev.set_expert(e, self.w1, self.w2, None, self.b1, self.b2, src_dtype=_lib.MOE_FP8_E4M3, s1=s1, s2=s2)
        elif self.w1.dtype == np.uint16:
            dev.set_expert(e, self.w1, self.w2, None, self.b1, self.b2, src_dtype=_lib.MOE_BF16)
        else:
            dev.set_expert(e, self.w1, self.w2, None, self.b1, self.b2, src_dtype=_lib.MOE_F32)

"""Activation functions of MixtureOfExperts.jl, as callables that also carry
the code the device epilogue implements.

Reference: ``silu(x) = x * sigmoid(x)`` (src/experts/gated.jl:35), NNlib's
``gelu`` (tanh form) as the ``MoEConfig.activation`` default
(src/core/moe_layer.jl:10), ``relu`` and ``identity``.  Calling one on a numpy
array evaluates the function elementwise (convenience for user code); the MoE
layer itself applies the activation on the device, fused into the expert GEMM
epilogue.
"""
import numpy as np

from . import _lib


class Activation:
    code = None
    name = ""

    def __call__(self, x):
        raise NotImplementedError

    def __repr__(self):
        return self.name


class _Silu(Activation):
    code = _lib.MOE_ACT_SILU
    name = "silu"

    def __call__(self, x):
        x = np.asarray(x, dtype=np.float32)
        return x / (np.float32(1) + np.exp(-x))


class _Gelu(Activation):
    code = _lib.MOE_ACT_GELU
    name = "gelu"

    def __call__(self, x):
        x = np.asarray(x, dtype=np.float32)
        c = np.float32(0.7978845608028654)
        return np.float32(0.5) * x * (np.float32(1) + np.tanh(c * (x + np.float32(0.044715) * x * x * x)))


class _Relu(Activation):
    code = _lib.MOE_ACT_RELU
    name = "relu"

    def __call__(self, x):
        return np.maximum(np.asarray(x, dtype=np.float32), np.float32(0))


class _Identity(Activation):
    code = _lib.MOE_ACT_IDENTITY
    name = "identity"

    def __call__(self, x):
        return np.asarray(x, dtype=np.float32)


silu = _Silu()
swish = silu  # NNlib.swish(x) = x * sigmoid(x)
gelu = _Gelu()
relu = _Relu()
identity = _Identity()


def activation_code(act):
    """Map an activation callable to the ABI enum; raise for anything else."""
    if isinstance(act, Activation):
        return act.code
    raise _lib.MoeError(
        _lib.MOE_EUNSUPPORTED,
        f"activation {act!r} has no device implementation (use silu, gelu, relu or identity)",
    )

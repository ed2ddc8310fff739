"""Activations (reference activations.py:19-67) as HIP kernels."""
import tl_hip as xp
import backend
from utils import Layer


class GeLU(Layer):
    """tanh-approximation GeLU, reference activations.py:19-28."""
    act_code = xp.TL_ACT_GELU

    def __init__(self):
        super(GeLU, self).__init__()

    def forward(self, input):
        self.input = input
        self.output = xp.activation(input, self.act_code)
        return self.output


class SiLU(Layer):
    """x * (1 + tanh(x/2)) / 2, reference activations.py:36-45."""
    act_code = xp.TL_ACT_SILU

    def __init__(self):
        super(SiLU, self).__init__()

    def forward(self, input):
        self.input = input
        self.output = xp.activation(input, self.act_code)
        return self.output


class SoftMax(Layer):
    """exp((x - max) / temperature) / sum over the last axis, reference
    activations.py:51-64. Padded rows (e.g. 50257-wide logits) keep their pitch."""

    def __init__(self, temperature=1.0):
        super(SoftMax, self).__init__()
        self.temperature = float(temperature)

    def forward(self, input):
        self.input = input
        self.output = xp.softmax(input, temperature=self.temperature)
        return self.output

    def backward(self, gradient):
        return gradient  # handled by the loss in the reference (activations.py:66-67)


def act_code_of(activation):
    """Activation class -> fused GEMM epilogue code, or None if it has no fused form."""
    return getattr(activation, "act_code", None)


__all__ = ["GeLU", "SiLU", "SoftMax", "act_code_of", "backend"]

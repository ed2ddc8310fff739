"""Inference driver (reference network.py:28-49: Network, predict/_forward, set_eval)."""
import tl_hip as xp
from utils import Layer

__all__ = ["Network"]


class Network:

    def __init__(self, layers: list[Layer]):
        self.layers = layers

    def predict(self, input):
        return self._forward(input)

    def _forward(self, input):
        for layer in self.layers:
            input = layer.forward(input)
        return input

    def set_eval(self, eval_mode):
        for layer in self.layers:
            layer.set_eval(eval_mode)

    def predict_ids(self, input):
        """argmax over the last axis of predict(input), as int64 on the device (the
        reference's `xp.argmax(y_hat, axis=-1)`, network.py:135, 158)."""
        return xp.argmax(self.predict(input), axis=-1)

    def train(self, *args, **kwargs):
        raise NotImplementedError("training is not part of the MI355X runtime")

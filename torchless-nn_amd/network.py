"""Inference driver (reference network.py:28-49: Network, predict/_forward, set_eval)."""
import tl_hip as xp
from utils import Layer

__all__ = ["Network", "CapturedForward"]


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

    def capture(self, example_input):
        """predict() captured once as a HIP graph for inputs shaped like `example_input`
        (not in the reference, which dispatches every op from Python each call,
        network.py:36-39): see CapturedForward."""
        return CapturedForward(self, example_input)


class CapturedForward:
    """A forward captured as one HIP graph. Each call copies the input into the captured
    input tensor (stream-ordered) and replays every kernel of the forward with one launch,
    then returns the captured output tensor: the same device tensor every call, rewritten
    by the next call, so read or copy it before calling again. destroy() (or garbage
    collection) frees the graph and the intermediates it holds."""

    def __init__(self, net, example_input):
        if not isinstance(example_input, xp.DeviceTensor):
            example_input = xp.array(example_input)
        self.net = net
        self.input = example_input.copy()
        net.predict(self.input)  # eager first: packed weights and scratch exist before capture
        with xp.capture() as cap:
            self.output = net.predict(self.input)
        self._graph = cap

    def __call__(self, input):
        if isinstance(input, xp.DeviceTensor):
            if input.shape != self.input.shape or input.dtype is not self.input.dtype:
                raise ValueError(f"captured for {self.input.shape} {self.input.dtype}, got "
                                 f"{input.shape} {input.dtype}")
            src = input if input.contiguous else input.copy()
            xp.copy_into(self.input, src)
        else:
            self.input.set(input)
        self._graph.launch()
        return self.output

    def destroy(self):
        self._graph.destroy()

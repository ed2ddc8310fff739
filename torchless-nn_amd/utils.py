"""Layer interface (reference utils.py:8-52).

Same attributes and methods as the reference. This runtime is inference-only, so
`register_param` records the parameter without allocating the gradient and AdamW state the
reference creates eagerly (utils.py:32-43): for the 2.5 B-parameter configurations those
would quadruple HBM use. `backward` raises.
"""


class Layer:

    def __init__(self):
        self.input = None
        self.output = None

        self.parameters = []
        self.gradients = []
        self.moments = []
        self.variances = []

        self.eval_mode = False
        self.is_embed_layer_back = False

    def forward(self, *input):
        raise NotImplementedError

    def backward(self, *input):
        raise NotImplementedError("training (backward) is not part of the MI355X runtime")

    def set_eval(self, eval_mode):
        self.eval_mode = eval_mode

    def register_param(self, parameter):
        self.parameters.append(parameter)
        return None

    def zero_grad(self):
        for grad in self.gradients:
            grad.fill(0)

    def zero_adam(self):
        for moment, variance in zip(self.moments, self.variances):
            moment.fill(0)
            variance.fill(0)

"""Pointwise MLP of the Transolver blocks (a caller of the hot path, not part
of it; reference ``flashslice/layers/basic.py:28-53``).

Module and parameter names are the reference's (``linear_pre``,
``linears``, ``linear_post``), so state dicts interchange with models built
from the reference package.
"""

import torch.nn as nn

# Activation factories by the reference's names (``basic.py:17-26``). The
# reference stores an *instance* for "leaky_relu", which its MLP then calls
# with no input; here every entry is a zero-argument factory, so "leaky_relu"
# builds LeakyReLU(0.1) like the others.
ACTIVATION = {
    "gelu": nn.GELU,
    "tanh": nn.Tanh,
    "sigmoid": nn.Sigmoid,
    "relu": nn.ReLU,
    "leaky_relu": lambda: nn.LeakyReLU(0.1),
    "softplus": nn.Softplus,
    "ELU": nn.ELU,
    "silu": nn.SiLU,
}


class MLP(nn.Module):
    """Linear -> act, ``n_layers`` x (Linear -> act, with a residual when
    ``res``), Linear. Unknown activations raise ``NotImplementedError``."""

    def __init__(self, n_input, n_hidden, n_output, n_layers=1, act="gelu", res=True):
        super().__init__()
        if act not in ACTIVATION:
            raise NotImplementedError("unknown activation %r" % (act,))
        make = ACTIVATION[act]
        self.n_input, self.n_hidden, self.n_output = n_input, n_hidden, n_output
        self.n_layers, self.res = n_layers, res
        # registration order (pre, post, hidden) fixes the order of the init
        # draws: the reference's, so one seed gives the same weights
        self.linear_pre = nn.Sequential(nn.Linear(n_input, n_hidden), make())
        self.linear_post = nn.Linear(n_hidden, n_output)
        self.linears = nn.ModuleList(
            nn.Sequential(nn.Linear(n_hidden, n_hidden), make()) for _ in range(n_layers))

    def forward(self, x):
        h = self.linear_pre(x)
        for block in self.linears:
            h = block(h) + h if self.res else block(h)
        return self.linear_post(h)

"""Model construction."""

from torch import nn

from fused_hoad.specs import MLPConfig

_ACTIVATIONS = {"tanh": nn.Tanh, "silu": nn.SiLU}


def build_mlp(config: MLPConfig) -> nn.Sequential:
    """``Linear, act`` repeated ``hidden_layers`` times, then ``Linear`` to ``output_dim``.

    Module order (and so the order of ``nn.Linear`` default initialisation draws under a given
    ``torch.manual_seed``) matches /root/reference/src/fused_hoad/models.py:15-26.
    """
    layers: list[nn.Module] = []
    width = config.input_dim
    for _ in range(config.hidden_layers):
        layers += [nn.Linear(width, config.hidden_dim), _ACTIVATIONS[config.activation]()]
        width = config.hidden_dim
    layers.append(nn.Linear(width, config.output_dim))
    return nn.Sequential(*layers)

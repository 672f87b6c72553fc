"""Shape contract of the MLP targeted by the fused kernels."""

from dataclasses import dataclass
from typing import Literal

ActivationName = Literal["tanh", "silu"]


@dataclass(frozen=True, slots=True)
class MLPConfig:
    """Dense MLP shape: ``input_dim -> hidden_dim x hidden_layers -> output_dim``."""

    input_dim: int
    hidden_dim: int
    hidden_layers: int
    output_dim: int = 1
    activation: ActivationName = "tanh"

    def __post_init__(self) -> None:
        for name in ("input_dim", "hidden_dim", "hidden_layers", "output_dim"):
            if getattr(self, name) < 1:
                raise ValueError(f"{name} must be positive")

"""Model shapes and numeric modes.

Shapes follow the GPT-2 base models named by the reference configs
(``model_config.base_model``): ``gpt2`` for pretrain_config/ablations/small.yaml:20,
``gpt2-medium`` for pretrain_config/medium.yaml:20.  ``large2x`` is the
double-parameter ablation shape used by the fp8 workload (32 layers at width
1280; the reference's large.yaml:20 names ``gpt2-large``, which has 36 layers on
the hub -- this build follows the 32-layer shape of its benchmark config).
All share GPT-2's 1024 learned positions, LayerNorm eps 1e-5, the tanh GELU,
a lm_head tied to the token embedding, and Conv1D weights stored ``[in, out]``.
"""
from __future__ import annotations

from dataclasses import dataclass, replace

from . import vocab

# numeric modes of the engine
FP32 = "float32"     # fp32 weights and activations: the fp32 check mode
BF16 = "bfloat16"    # bf16 weights, bf16 GEMM operands, fp32 residual stream
FP8W = "fp8w"        # fp8 e4m3 per-output-channel weights, bf16 activations
MODES = (FP32, BF16, FP8W)


@dataclass(frozen=True)
class ModelConfig:
    n_layer: int
    d_model: int
    n_head: int
    vocab_size: int = vocab.VOCAB_SIZE
    n_positions: int = 1024
    max_length: int = vocab.MAX_LENGTH
    eps: float = 1e-5

    @property
    def head_dim(self) -> int:
        return self.d_model // self.n_head

    @property
    def d_ff(self) -> int:
        return 4 * self.d_model

    @property
    def linear_params(self) -> int:
        """Weights of the four Conv1D GEMMs over all layers (12 L d^2)."""
        return 12 * self.n_layer * self.d_model * self.d_model

    def with_(self, **kw) -> "ModelConfig":
        return replace(self, **kw)


SMALL = ModelConfig(n_layer=12, d_model=768, n_head=12)
MEDIUM = ModelConfig(n_layer=24, d_model=1024, n_head=16)
LARGE2X = ModelConfig(n_layer=32, d_model=1280, n_head=20)
TINY = ModelConfig(n_layer=2, d_model=256, n_head=4)  # tests only

PRESETS = {"small": SMALL, "medium": MEDIUM, "large2x": LARGE2X, "tiny": TINY}

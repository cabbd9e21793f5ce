"""Fused LM head (lm_head GEMM + cross-entropy + entropy + argmax) on the HIP row kernel
esep_head_row_softmax, with the reference's solution/head API (fused_linear_ce, warmup).

The reference's trainer integration (solution/head/patch.py: Qwen2ForCausalLM / TRL SFTTrainer /
Soup wiring) is not provided: TRL and Soup are not part of this build, and the integration is
outside the kernel path.
"""

from .op import CHUNK_ROWS, G_SCALE, VOCAB, FusedLinearCE, fused_linear_ce, warmup

__all__ = ["fused_linear_ce", "FusedLinearCE", "warmup", "CHUNK_ROWS", "G_SCALE", "VOCAB"]

"""MI355X-native rebuild of the decoder-body hot path of gojosatorukz/esep-soup-kernels.

solution.body: fused residual-add + RMSNorm and RoPE (the hot path), varlen attention, the LoRA
dropout kernels and the packed Qwen2 layer; solution.swiglu: the SwiGLU MLP activation;
solution.nf4: NF4 double-quant dequantization; solution.head: the fused LM head
(fused_linear_ce). All compute runs in libesep_body.so (HIP, gfx950). The reference's startup
patches and trainer integrations are not part of this package. `apply()` installs the body
patch, as the reference's solution/__init__.py:19-25 does for what exists here.
"""


def apply():
    from .body import patch as patch_body

    patch_body()

"""MI355X-native rebuild of the decoder-body hot path of gojosatorukz/esep-soup-kernels.

solution.body: fused residual-add + RMSNorm and RoPE (the hot path), varlen attention, the LoRA
dropout kernels and the packed Qwen2 layer; solution.swiglu: the SwiGLU MLP activation;
solution.nf4: NF4 double-quant dequantization; solution.head: the fused LM head
(fused_linear_ce). All compute runs in libesep_body.so (HIP, gfx950). The reference's startup
patches and trainer integrations are not part of this package. `apply()` installs the SwiGLU
and body patches, as the reference's solution/__init__.py:19-25 does for what exists here.
"""


def apply():
    """Install the patches this package provides, in the reference's order
    (solution/__init__.py:19-25): Qwen2MLP on the HIP SwiGLU, then the packed decoder body. The
    reference's other steps have nothing to act on here: its Triton warmup thread and startup
    patch (HIP is compiled ahead of time), the bitsandbytes Linear4bit patch (bitsandbytes is
    absent; solution.nf4 exposes the dequantization and the linear directly) and the TRL / Soup
    LM-head patch (solution.head exposes fused_linear_ce)."""
    from .swiglu import patch_qwen2_mlp

    patch_qwen2_mlp()
    from .body import patch as patch_body

    patch_body()

"""MI355X-native rebuild of the decoder-body hot path of gojosatorukz/esep-soup-kernels.

Only the body workstream's RMSNorm / RoPE path is provided (solution.body); the reference's
other workstreams (NF4 dequant, LM head, LoRA dropout, startup patches) are not part of this
package. `apply()` installs what exists, as the reference's solution/__init__.py:19-25 does.
"""


def apply():
    from .body import patch as patch_body

    patch_body()

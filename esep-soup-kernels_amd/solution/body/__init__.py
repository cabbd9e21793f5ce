"""Workstream `body`: the Qwen2 decoder body's RMSNorm and rotary-embedding kernels (HIP,
gfx950) and the packed-decoder patch point that routes HF Qwen2 through them.

Reference: solution/body/__init__.py:10-22 (patch, warmup).
"""


def patch():
    """Install the body patches (class-patches Qwen2Model.forward). Safe to call more than once."""
    from .packed import patch as patch_packed

    patch_packed()


def warmup(device=None):
    """Load libesep_body.so ahead of the first step. The kernels are compiled ahead of time
    (build.py), so unlike the reference's Triton warmup (body/warmup.py) nothing is compiled
    here; never raises, as the reference's warmup does not."""
    try:
        from . import _hip

        _hip.lib()
    except Exception:  # noqa: BLE001 - warmup is best effort, errors resurface at first use
        pass

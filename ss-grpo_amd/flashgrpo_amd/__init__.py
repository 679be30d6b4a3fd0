"""flashgrpo_amd: MI355X-native FlashGRPO speculative rollout step.

Mirrors the reference's ``flashgrpo.decoding`` / ``flashgrpo.models`` API
(ihbkaiser/ss-GRPO) on top of hand-written gfx950 HIP kernels reached through
a C ABI (``include/flashgrpo_amd.h``, loaded with ctypes by ``_lib``).
"""
__version__ = "0.1.0"

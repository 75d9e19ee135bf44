"""MI355X (gfx950) SuffixGPU drafter.

Drop-in for zip95297/SuffixGPU's draft path (suffix_gpu/__init__.py:1-4):
``SuffixGPUDrafter`` with propose / update_state / propose_with_update /
harvest_finished / poll, running hand-written HIP kernels from
``libsuffixgpu_amd.so`` (built by ``python -m suffixgpu_amd.build``).
"""

from suffixgpu_amd.proposer import SuffixGPUDrafter

__version__ = "0.1.2"
__all__ = ["SuffixGPUDrafter", "__version__"]

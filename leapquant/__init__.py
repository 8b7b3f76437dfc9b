"""LeapQuant's INT8 recurrent-state decode path under the reference's own import name.

``leapquant.kernels``, ``leapquant.state`` and ``leapquant.vllm`` are the modules of the MI355X implementation in
``leapquant_amd`` -- the same module objects, so ``from leapquant.state import get_state`` and the vLLM entry point
``leapquant.vllm:register`` (/root/reference/pyproject.toml:14-15) reach the same per-layer registry and kernels as
``leapquant_amd.state`` does.  Nothing here computes.
"""
import sys

import leapquant_amd
from leapquant_amd import kernels, state, vllm
from leapquant_amd.vllm import gdn as _gdn, glm as _glm

__version__ = leapquant_amd.__version__

for _name, _mod in (("kernels", kernels), ("state", state), ("vllm", vllm), ("vllm.gdn", _gdn), ("vllm.glm", _glm)):
    sys.modules[__name__ + "." + _name] = _mod
del _name, _mod

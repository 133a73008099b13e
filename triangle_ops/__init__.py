"""`import triangle_ops` resolves to triangleops_amd, under the reference package's import name.

Every submodule (`triangle_ops.triangle_mul`, `triangle_ops.triangle_attn.kernel`,
`triangle_ops._common`, ...) is the same module object as its `triangleops_amd` counterpart,
so code written against the reference package runs unchanged.
"""

import sys as _sys

import triangleops_amd as _impl
from triangleops_amd import *  # noqa: F401,F403
from triangleops_amd import __all__, __version__  # noqa: F401

for _name, _mod in list(_sys.modules.items()):
    if _name.startswith("triangleops_amd."):
        _sys.modules["triangle_ops." + _name[len("triangleops_amd."):]] = _mod
        globals().setdefault(_name.split(".")[1], getattr(_impl, _name.split(".")[1]))

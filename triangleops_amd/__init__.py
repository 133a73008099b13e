"""triangleops_amd — AlphaFold-3 Pairformer primitives as hand-written gfx950 (MI355X) kernels.

Drop-in for the `triangle_ops` Python API of youngchan2/TriangleOps (reference
`triangle_ops/__init__.py:17-31`): the same three op modules and one-shot functions, each
with `precompute(...)` (one-time weight folding -> dict), `forward(x, pre, ...)` (per call)
and a one-shot `<op_name>(...)`:

    attention_pair_bias            QKV proj + LN(Z) bias proj + attention, then gate + W_o
    triangle_attention             LN + bias proj, Q/K/V proj + attention, then gate + W_o
    triangle_multiplicative_update LN + gated proj, triangle einsum, LN + gated proj

`attn_pair_bias.attention_pair_bias_qknorm` adds the K-Fold variant the reference states only in
torch (`benchmarks/references.py:230-277`: Q bias, LayerNorm over H*D of Q and K, key mask), and
`pairformer` composes the ops into a Pairformer block's pair stack and single update with the
residual adds fused into the output kernels, and `graph.capture` replays a fixed-shape call as
one HIP graph (for the launch-bound small sizes).

All compute runs in `libtriangleops_amd.so` (HIP, gfx950) through a C ABI
(`include/triangleops_amd.h`); there is no CPU or fallback path.
"""

from . import attn_pair_bias, graph, pairformer, triangle_attn, triangle_mul
from .attn_pair_bias import attention_pair_bias
from .triangle_attn import triangle_attention
from .triangle_mul import triangle_multiplicative_update

__version__ = "0.1.0"

__all__ = [
    "attn_pair_bias",
    "triangle_attn",
    "triangle_mul",
    "attention_pair_bias",
    "triangle_attention",
    "triangle_multiplicative_update",
]

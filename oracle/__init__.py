"""CPU oracle for the MoE-LoRA expert layer.  TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the arithmetic of the path that ART's
Megatron GRPO backend trains (router -> top-k softmax / routing replay ->
expert-major permute -> grouped SwiGLU expert FC1/FC2 with frozen base weights
plus per-expert LoRA -> un-permute/combine), forward and backward.

It is the checker, never the thing measured or shipped.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it.  The product package (``art-mlx_amd/art_amd``) must never import it
and fails loudly when its HIP library is missing.

Modules
-------
``oracle.routing``  numpy restatement of the integer routing work: top-k with
                    the documented tie rule, renormalised softmax, replay
                    gather, and the expert-major / token-ascending dispatch
                    plan (counts, offsets, destination rows, row -> token).
``oracle.layer``    torch-CPU (fp32 or fp64) restatement of the float work:
                    router gating linear, grouped base linears, grouped LoRA
                    (single and dual), weighted SwiGLU, permute / un-permute,
                    and the full layer, differentiated by torch autograd.

Pinning (what checks each function against something other than itself) is
listed in each module's header; functions with no independent check say
"parity unpinned".
"""

"""MI355X (gfx950) TriS-MoE grouped expert dequant-GEMM path.

The compute lives in ``libtris_moe_hip.so`` (hand-written HIP kernels behind
the C ABI in ``include/tris_moe_hip.h``); this package is the host side that
mirrors the reference's Python interface for the path:

* ``ext``      — drop-in for the native module ``autogptq_TriS_cuda``
  (grouped entry points, same names and argument order);
* ``qlinear``  — ``build_grouped_route``, ``run_grouped_structured_expert_forward``,
  ``run_grouped_structured_expert_pair_forward``, payload stacking,
  ``QuantLinear`` / ``ExpertSharedMatrix`` (``qlinear_cuda.py``);
* ``moe``      — the sparse MoE block (``modeling_mixtral.py``);
* ``synthetic``/``configs`` — seeded payloads of the BASELINE configurations;
* ``packing``  — payload bit/half layouts (``utils/pack_utils.py``).
"""
from ._lib import TRIS_COMPACT3_KERNEL_ABI_VERSION, TrisExtensionUnavailable, load as load_library  # noqa: F401

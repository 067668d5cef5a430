"""MI355X (gfx950) DeepSeek-V4-Flash MoE expert hot path.

Host side of a HIP library (``libdsv4moe.so``, C ABI in ``include/dsv4moe.h``)
that replaces gaiban-lite's ``runtime/dsv4_direct`` MoE layer: router,
deterministic alignment, grouped int4 expert GEMMs with the SwiGLU epilogue,
routing-weighted combine and the shared expert.

The directory name is not a Python identifier, so importing it registers the
alias ``gaiban_lite_amd`` (and aliases for every submodule) in ``sys.modules``:

    import importlib; importlib.import_module("gaiban-lite_amd")
    from gaiban_lite_amd import TP4MoE
"""

from __future__ import annotations

import sys

from . import _lib, build_ext, contracts, linear_plan, ops, synthetic, weights  # noqa: F401
from . import checkpoint, deterministic_moe_align, fixed_moe_align, fp8_linear, moe_forward, moe_runtime  # noqa: F401
from . import weight_only_linear  # noqa: F401
from .deterministic_moe_align import (  # noqa: F401
    DeterministicMoEAlignment,
    allocate_deterministic_moe_alignment,
    deterministic_moe_align_block_size,
    max_padded_tokens,
)
from .moe_forward import (  # noqa: F401
    GateForwardTensors,
    HashGateForwardTensors,
    error_metrics,
    gate_forward,
    gate_forward_with_boundary,
    gate_logits,
    hash_gate_forward,
    route_from_logits,
)
from .moe_runtime import (  # noqa: F401
    MoELayer,
    MoERouteCaptureBuffer,
    MoERouteCaptureEvidence,
    MoERouteOverride,
    MoERouteTensors,
    MoETrace,
    ResidentGateWeights,
    TP4MoE,
    TP4MoEConfig,
)
from .weights import (  # noqa: F401
    ResidentFP8SharedExpert,
    ResidentInt4MoEWeights,
    ResidentMXFP4MoEWeights,
    int4_g128_expert_bytes,
    mxfp4_g32_expert_bytes,
)

ALIAS = "gaiban_lite_amd"


def _register_alias() -> None:
    me = sys.modules[__name__]
    sys.modules.setdefault(ALIAS, me)
    prefix = __name__ + "."
    for name, mod in list(sys.modules.items()):
        if name.startswith(prefix):
            sys.modules.setdefault(ALIAS + "." + name[len(prefix):], mod)


_register_alias()

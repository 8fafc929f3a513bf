"""MI355X-native FP8 block-scaled packed MoE path of kiojuvr/glm53-flash-mlx.

Import as ``importlib.import_module("glm53-flash-mlx_amd")`` with the
repository root on ``sys.path``.  The compute path is libglm53_moe.so (HIP,
gfx950) behind the C ABI of include/glm53_moe.h; this package is the host
mirror of the reference's fp8.py / packed.py / grouped_fp8.py / loader.py
interface for that path.
"""

from .abi import (
    GROUPED_KERNEL_ABI,
    GROUPED_MEASURED_CROSSOVER_ROUTES,
    GROUPED_MIN_ROUTES,
    KERNEL_ABI_VERSION,
    PACKED_DECODE_KERNEL_ABI,
    PACKED_EXPERT_BANK_ABI,
)
from .checkpoint import CheckpointError, load_moe_layer
from .fp8 import (
    BLOCK_SIZE,
    DECODE_TOP_K,
    BlockFP8Linear,
    ClampedMLP,
    DirectFP8Expert,
    DirectFP8MoE,
    block_fp8_linear,
    swiglu,
)
from .grouped_fp8 import (
    GROUPED_TILE_ROWS,
    PrefillPlan,
    SortedGroupedFP8MoE,
    activate_gate_up,
    build_grouped_tile_plan,
    build_route_plan,
    grouped_fp8_linear,
    restore_and_reduce,
)
from .loader import install_packed_decode_moe, install_packed_grouped_moe, install_packed_moe
from .ownership import (
    ResidentTensor,
    TensorLayout,
    TensorLease,
    TensorOwnership,
    TensorOwnershipError,
    borrowed_ephemeral_tensor,
    borrowed_stable_tensor,
    materialize_owned,
    owned_tensor,
    require_resident,
    resident_concatenate,
)
from .packed import BankHandle, DecodePlan, PackedFP8ExpertBank, PackedFP8MoE, RoutedDiagnostic
from .router import Float32Gate

__all__ = [
    "CheckpointError",
    "load_moe_layer",
    "BLOCK_SIZE", "DECODE_TOP_K", "GROUPED_TILE_ROWS", "GROUPED_MIN_ROUTES", "GROUPED_MEASURED_CROSSOVER_ROUTES",
    "KERNEL_ABI_VERSION", "GROUPED_KERNEL_ABI", "PACKED_EXPERT_BANK_ABI", "PACKED_DECODE_KERNEL_ABI",
    "block_fp8_linear", "swiglu", "BlockFP8Linear", "ClampedMLP", "DirectFP8Expert", "DirectFP8MoE",
    "PackedFP8ExpertBank", "PackedFP8MoE", "DecodePlan", "Float32Gate", "build_route_plan",
    "build_grouped_tile_plan", "grouped_fp8_linear", "activate_gate_up", "restore_and_reduce",
    "SortedGroupedFP8MoE", "PrefillPlan", "install_packed_moe", "install_packed_grouped_moe",
    "install_packed_decode_moe", "BankHandle", "RoutedDiagnostic", "ResidentTensor", "TensorLayout", "TensorLease", "TensorOwnership",
    "TensorOwnershipError", "borrowed_ephemeral_tensor", "borrowed_stable_tensor", "materialize_owned",
    "owned_tensor", "require_resident", "resident_concatenate",
]

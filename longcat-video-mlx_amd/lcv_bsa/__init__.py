"""lcv_bsa -- Block Sparse Attention forward for MI355X (gfx950).

A ``backend="hip"`` for LongCat-Video's BSA: the reference API
(``bsa_attention``, its helpers, the kernel-level ``bsa_attention_hip``, the
``_process_attn`` dispatcher and ``enable_bsa``) on PyTorch-ROCm tensors, with
the arithmetic in hand-written gfx950 kernels behind the C ABI declared in
``include/lcv_bsa.h``.
"""

from .block_sparse_attention import (  # noqa: F401
    block_routing_scores,
    bsa_attention,
    build_token_block_indices,
    build_token_pair_mask,
    mean_pool_blocks_3d,
    num_blocks,
    num_selected_blocks,
    select_block_indices,
    topk_block_indices,
)
from .block_sparse_attention_hip import (  # noqa: F401
    bsa_attention_hip,
    schedule_block_order,
    reshape_from_block_major,
    reshape_to_block_major,
)
from .prepare import prepare_qk, rope_table  # noqa: F401
from .attention import BSAAttention, backend_from_env  # noqa: F401
from .dit import BSAModelMixin, apply_bsa_params, disable_bsa, enable_bsa  # noqa: F401

__version__ = "0.1.0"

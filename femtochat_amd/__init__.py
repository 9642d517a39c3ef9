"""MI355X-native flash attention for femtochat (forward and backward).

The compute path is libfemtochat_attn.so (hand-written gfx950 HIP kernels
behind a C ABI, include/femtochat_attn.h); ``femtochat_amd.kernels`` is the
host-side mirror of the reference's ``Kernels`` attention API, and
``femtochat_amd.prologue`` the rotary embedding + RMS norm that
``CausalSelfAttention`` applies to Q and K before it, and
``femtochat_amd.loss`` the cross-entropy and token-embedding kernels either
side of the model (include/femtochat_loss.h), ``femtochat_amd.optim`` the
optimizer kernels (include/femtochat_optim.h).
"""
from .kernels import (  # noqa: F401
    AttentionFunction,
    AttentionState,
    MFMAExact,
    MFMAFast,
    accumulator_type,
    attention,
    attention_,
    attention_inputs,
    attention_state,
    backward_workspace_bytes,
    forward_workspace_bytes,
    capabilities,
    convert_,
    delta_attention_,
    fill_zero_,
    instruction,
    window_sizes,
)
from .prologue import (  # noqa: F401
    AttentionPrologueFunction,
    attention_prologue,
    attention_prologue_,
    delta_attention_prologue_,
    rotary_embeddings,
)
from .loss import (  # noqa: F401
    CrossEntropyFunction,
    EmbeddingFunction,
    cross_entropy,
    cross_entropy_,
    cross_entropy_fused_,
    cross_entropy_gradient_,
    embedding,
    embedding_,
    embedding_gradient_,
    valid_target_count,
)
from .optim import (  # noqa: F401
    AdamW,
    adam_update_,
    adamw_step_,
    gather_,
    muon_update_,
    polar_express,
    polar_express_,
    scatter_,
)

__version__ = "0.1.0"

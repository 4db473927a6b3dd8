"""suika_amd -- MI355X-native reshard engine for Suika's live state migration.

Public API mirrors the reference's migration module (Suika/migration.py):
``TensorMeta``, ``ParamLayout``, ``TransferOp``, ``schedule_param_transfer``,
``execute_param_transfer``, ``schedule_and_execute_param_transfer``,
``merge_model_and_optimizer_state_dict``, ``split_model_and_optimizer_state_dict``,
``checkpoint_save``, ``checkpoint_load``, ``migration_save``, ``migration_load``, and
the helpers ``forcefully_free_tensor`` / ``cuda_gc`` (Suika/utils.py:248-260).
The data movement runs in HIP kernels behind the C ABI of
``lib/libsuika_reshard.so`` (include/suika_reshard.h).
"""
from .meta import (CHUNK, QKV_HEADS, VOCAB_PAD, ParamLayout, TensorMeta, TransferOp,
                   get_named_parameters_and_persistent_buffers, get_param_tensor_meta,
                   schedule_param_transfer, vocab_padded)
from .migration import (cuda_gc, execute_param_transfer, forcefully_free_tensor,
                        merge_model_and_optimizer_state_dict, schedule_and_execute_param_transfer,
                        split_model_and_optimizer_state_dict)
from .plan import PlanOptions, ReshardPlan, SlotSpec
from ._lib import PlanError, ReshardError
from .checkpoint import checkpoint_load, checkpoint_save, migration_load, migration_save
from .handoff import HandoffError, dummy_migration_IPC_state_dict

__all__ = [
    "CHUNK", "QKV_HEADS", "VOCAB_PAD", "ParamLayout", "TensorMeta", "TransferOp",
    "get_named_parameters_and_persistent_buffers", "get_param_tensor_meta",
    "schedule_param_transfer", "vocab_padded", "execute_param_transfer",
    "merge_model_and_optimizer_state_dict", "schedule_and_execute_param_transfer",
    "split_model_and_optimizer_state_dict", "PlanOptions", "ReshardPlan", "SlotSpec",
    "PlanError", "ReshardError", "checkpoint_save", "checkpoint_load", "migration_save",
    "migration_load", "forcefully_free_tensor", "cuda_gc", "dummy_migration_IPC_state_dict", "HandoffError",
]

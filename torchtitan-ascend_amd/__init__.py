"""MI355X-native MoE expert path with the converter surface of torchtitanturbo.

Drop-in for the two converters the reference registers
(torchtitanturbo/models/llama4/config_registry.py:52-57):

    NpuGroupedExpertsConverter.Config()  ->  HipGroupedExpertsConverter.Config()
    NpuTokenDispatcherConverter.Config() ->  HipTokenDispatcherConverter.Config()

The directory name is not a Python identifier; import it with
`importlib.import_module("torchtitan-ascend_amd")`.  Importing it has no
side effects: nothing is patched, nothing is loaded until an op runs.
"""
from .functional import HIPMoeTokenUnpermute, moe_experts_forward, run_experts_grouped_mm
from .grouped_experts import HipGroupedExperts, HipGroupedExpertsConverter
from .protocol import HAVE_TORCHTITAN
from . import state_dict
from .token_dispatcher import HipDispatchMetadata, HipTokenDispatcher, HipTokenDispatcherConverter

__all__ = [
    "HAVE_TORCHTITAN",
    "HIPMoeTokenUnpermute",
    "HipDispatchMetadata",
    "HipGroupedExperts",
    "HipGroupedExpertsConverter",
    "HipTokenDispatcher",
    "HipTokenDispatcherConverter",
    "moe_experts_forward",
    "run_experts_grouped_mm",
    "state_dict",
]

"""chomikgrad API surface with an MI355X-native ``hip`` compiler plugin.

Registration follows the reference (chomikgrad/__init__.py:41-45): the
plugin is registered by class, so importing this package never touches a
device; the first ``get_compiler("hip")`` loads ``libchomik_hip.so``.
"""

from .dtypes import BFLOAT16
from .generation import (
    GreedyVerification,
    verify_greedy_block_with_bonus,
    verify_greedy_candidates,
)
from .hip_backend import HIPArray, HIPCompiler, HIPDeviceAdapter, HIPProgram, register_into
from .lazy import (
    CompiledProgram,
    Compiler,
    DeviceAdapter,
    GraphPlan,
    LazyNode,
    Op,
    get_compiler,
    realize_nodes,
    register_compiler,
    set_default_compiler,
    topological_sort,
)
from .llama import (
    LlamaBatchedDecoderStep,
    LlamaConfig,
    LlamaDecoderBlock,
    LlamaDecoderStep,
    LlamaForCausalLM,
)
from .tensor import Tensor, compile_graph, no_grad, realize

register_compiler("hip", HIPCompiler)

__all__ = [
    "BFLOAT16",
    "CompiledProgram",
    "Compiler",
    "DeviceAdapter",
    "GraphPlan",
    "GreedyVerification",
    "HIPArray",
    "HIPCompiler",
    "HIPDeviceAdapter",
    "HIPProgram",
    "LazyNode",
    "LlamaBatchedDecoderStep",
    "LlamaConfig",
    "LlamaDecoderBlock",
    "LlamaDecoderStep",
    "LlamaForCausalLM",
    "Op",
    "Tensor",
    "compile_graph",
    "get_compiler",
    "no_grad",
    "realize",
    "realize_nodes",
    "register_into",
    "register_compiler",
    "set_default_compiler",
    "topological_sort",
    "verify_greedy_block_with_bonus",
    "verify_greedy_candidates",
]

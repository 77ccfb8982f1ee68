"""The hip plugin registered into another copy of the plugin API.

The reference's registry (chomikgrad/lazy.py:646-678) accepts a compiler
only if it is an instance of *its own* ``Compiler`` ABC, and its graphs are
made of *its own* ``LazyNode`` objects whose ``op`` is *its own* ``Op`` enum
(lazy.py:22-104).  ``foreign_api()`` builds a stand-in with exactly those
properties: a second ``Op`` class with the reference's member names and
values, a node class with the reference's slots, the three plugin ABCs and
a registry with the reference's checks.  Graphs converted into it must plan
to the same tape as the native graph, and ``register_into`` must make the
plugin acceptable to that registry.
"""

from __future__ import annotations

import types
from abc import ABC, abstractmethod
from enum import Enum

import numpy as np
import pytest

from chomikgrad import Tensor, realize, register_into, synthetic
from chomikgrad._planner import plan_graph
from chomikgrad.hip_backend import HIPCompiler
from chomikgrad.llama import LlamaConfig, LlamaDecoderStep, _rope_rotations, decode_masks
from tape_model import CpuPlanCompiler, run


def foreign_api() -> types.ModuleType:
    module = types.ModuleType("foreign_lazy")

    class Op(Enum):  # same names and values as lazy.py:22-34, another class
        ELEMENTWISE = "elementwise"
        REDUCE = "reduce"
        RESHAPE = "reshape"
        PERMUTE = "permute"
        MATMUL = "matmul"
        GATHER = "gather"

    class LazyNode:  # the slots of lazy.py:37-104
        __slots__ = ("op", "inputs", "arg", "shape", "dtype", "value", "native_values",
                     "cache_native", "lowering")

        def __init__(self, op, inputs, arg, shape, dtype, value=None, native_values=None,
                     cache_native=True, lowering=None):
            self.op, self.inputs, self.arg = op, tuple(inputs), arg
            self.shape, self.dtype, self.value = tuple(shape), np.dtype(dtype), value
            self.native_values = native_values or {}
            self.cache_native, self.lowering = cache_native, lowering

        def numpy_value(self):
            if self.value is None:
                backend, native = next(iter(self.native_values.items()))
                self.value = np.array(module.get_compiler(backend).device.to_numpy(native), copy=True)
            return self.value

    class DeviceAdapter(ABC):
        @abstractmethod
        def array(self, value): ...

    class CompiledProgram(ABC):
        @abstractmethod
        def run(self, bindings=None, *, synchronize=False): ...

    class Compiler(ABC):
        @abstractmethod
        def compile(self, outputs, dynamic_inputs=()): ...

    registry, instances = {}, {}

    def register_compiler(name, compiler, *, replace=False):  # lazy.py:646-656
        if name in registry and not replace:
            raise ValueError(f"compiler already registered: {name}")
        if not isinstance(compiler, Compiler) and not callable(compiler):
            raise TypeError("compiler must be a Compiler instance or a factory")
        registry[name] = compiler
        instances.pop(name, None)

    def get_compiler(name):  # lazy.py:666-678
        if name in instances:
            return instances[name]
        registration = registry[name]
        compiler = registration() if callable(registration) else registration
        if not isinstance(compiler, Compiler):
            raise TypeError(f"compiler factory {name!r} returned an invalid object")
        instances[name] = compiler
        return compiler

    module.__dict__.update(Op=Op, LazyNode=LazyNode, DeviceAdapter=DeviceAdapter,
                           CompiledProgram=CompiledProgram, Compiler=Compiler,
                           register_compiler=register_compiler, get_compiler=get_compiler,
                           registry=registry)
    return module


def convert(outputs, api):
    """Rebuild a graph of this package's nodes as ``api`` nodes (op by value),
    keeping leaf values, natives and lowering tags; returns (outputs, map)."""
    mapping = {}

    def visit(node):
        if node in mapping:
            return mapping[node]
        inputs = tuple(visit(parent) for parent in node.inputs)
        lowering = None
        if node.lowering is not None:
            kind, parents, argument = node.lowering
            lowering = (kind, tuple(visit(parent) for parent in parents), argument)
        op = None if node.op is None else api.Op(node.op.value)
        mapping[node] = api.LazyNode(op, inputs, node.arg, node.shape, node.dtype, node.value,
                                     dict(node.native_values), node.cache_native, lowering)
        return mapping[node]

    return [visit(node) for node in outputs], mapping


def decode_graph(dtype=np.float16):
    config = LlamaConfig(vocab_size=256, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                         num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=64)
    weights = synthetic.weights_as_tensors(synthetic.host_weights(config, dtype, seed=5))
    C, position = 40, 21
    attention, write = decode_masks(position, C, dtype)
    leaves = [Tensor(np.array([[7]], np.int32), copy=False),
              Tensor(_rope_rotations(1, 64, config.rope_theta, dtype, offset=position), copy=False),
              Tensor(attention, copy=False), Tensor(write, copy=False),
              Tensor(np.asarray(position, np.int32), copy=False)]
    rng = np.random.default_rng(6)
    caches = [Tensor(rng.normal(0, 0.5, (1, 2, C, 64)).astype(dtype), copy=False) for _ in range(4)]
    step = LlamaDecoderStep(config, weights, cache_length=C, dtype=dtype)
    outputs = step(*leaves[:4], list(zip(caches[::2], caches[1::2])), position=leaves[4])
    return outputs, leaves + caches


def test_foreign_nodes_plan_to_the_same_tape_and_values():
    outputs, dynamic = decode_graph()
    nodes = [t._node for t in outputs]
    dyn = [t._node for t in dynamic]
    native = plan_graph(CpuPlanCompiler(), nodes, dyn, dyn[5:])
    api = foreign_api()
    foreign_outputs, mapping = convert(nodes, api)
    foreign = plan_graph(CpuPlanCompiler(), foreign_outputs, [mapping[n] for n in dyn],
                         [mapping[n] for n in dyn[5:]])
    assert foreign.source == native.source
    assert np.array_equal(foreign.tape, native.tape)
    # Same fused kernels: the Llama rewrites matched the foreign op values.
    assert "decode_attention" in foreign.source and "gemv[rms_norm+silu_mul]" in foreign.source
    values = {leaf: leaf.numpy_value() for leaf in native.input_slots}
    got_native = run(native, values)
    got_foreign = run(foreign, {mapping[leaf]: value for leaf, value in values.items()})
    for a, b in zip(got_native, got_foreign):
        assert np.array_equal(a, b)
    expected = realize(*outputs, compiler="cpu")
    np.testing.assert_allclose(got_foreign[0].astype(np.float32), expected[0].astype(np.float32),
                               atol=2e-2, rtol=1e-2)


def test_register_into_a_foreign_registry():
    api = foreign_api()
    register_into(api)
    assert api.registry["hip"] is HIPCompiler
    assert issubclass(HIPCompiler, api.Compiler)
    with pytest.raises(ValueError):
        register_into(api)  # duplicate names raise unless replace=True (lazy.py:650-651)
    register_into(api, replace=True)


@pytest.mark.gpu
def test_foreign_registry_runs_on_the_gpu(hip):
    """End to end through the foreign registry: get_compiler("hip") passes its
    isinstance check, compiles the foreign graph and runs it on the device."""
    print("[gpu case] foreign registry decode step", flush=True)
    outputs, dynamic = decode_graph()
    api = foreign_api()
    register_into(api)
    compiler = api.get_compiler("hip")
    assert isinstance(compiler, api.Compiler)
    foreign_outputs, mapping = convert([t._node for t in outputs], api)
    program = compiler.compile(foreign_outputs, [mapping[t._node] for t in dynamic])
    assert isinstance(program, api.CompiledProgram) and isinstance(program.device, api.DeviceAdapter)
    got = program()
    expected = realize(*outputs, compiler="cpu")
    np.testing.assert_allclose(got[0].astype(np.float32), expected[0].astype(np.float32), atol=2e-2, rtol=1e-2)
    # Cache rows other than the written position are returned bit for bit;
    # the written row holds RoPE(k) / v from the GEMV, within float16 noise.
    written = 21
    for value, reference in zip(got[1:], expected[1:]):
        keep = np.arange(value.shape[2]) != written
        assert np.array_equal(value[:, :, keep], reference[:, :, keep])
        np.testing.assert_allclose(value[:, :, written].astype(np.float32),
                                   reference[:, :, written].astype(np.float32), atol=2e-2, rtol=1e-2)

"""Converter surface (CPU).  Mirrors the reference's interface tests
(tests/unit_tests/test_converters.py:14-125) for the Hip converters, plus
the conversion semantics of npu_gmm.py:130-152 and npu_permute.py:102-117."""
from __future__ import annotations

import dataclasses
import importlib

import pytest
import torch

pkg = importlib.import_module("torchtitan-ascend_amd")
P = importlib.import_module("torchtitan-ascend_amd.protocol")
CONVERTERS = [pkg.HipGroupedExpertsConverter, pkg.HipTokenDispatcherConverter]


@pytest.mark.parametrize("conv", CONVERTERS)
def test_converter_has_dataclass_config(conv):
    assert hasattr(conv, "Config") and dataclasses.is_dataclass(conv.Config)
    assert isinstance(conv.Config(), P.ModelConfigConverter.Config)


@pytest.mark.parametrize("conv", CONVERTERS)
def test_converter_initialises_with_empty_config(conv):
    c = conv(conv.Config())
    assert isinstance(c, conv)
    assert callable(c.convert)
    assert isinstance(conv.Config().build(), conv)


def test_converter_naming():
    for conv, module in ((pkg.HipGroupedExpertsConverter, pkg.HipGroupedExperts),
                         (pkg.HipTokenDispatcherConverter, pkg.HipTokenDispatcher)):
        assert conv.__name__.endswith("Converter")
        assert conv.__name__ == module.__name__ + "Converter"


def _model(score_before=True, K=1, E=8):
    mc = P.ModelConfig()
    disp = P.AllToAllTokenDispatcher.Config(num_experts=E, top_k=K, score_before_experts=score_before)
    mc.layers = [
        P.GroupedExperts.Config(dim=256, hidden_dim=512, num_experts=E, token_dispatcher=disp),
        P.GroupedExperts.Config(dim=256, hidden_dim=512, num_experts=E,
                                token_dispatcher=P.AllToAllTokenDispatcher.Config(num_experts=E, top_k=K)),
    ]

    @dataclasses.dataclass
    class Block:
        moe: object

    mc.block = Block(moe=P.GroupedExperts.Config(dim=128, hidden_dim=256, num_experts=E, token_dispatcher=disp))
    return mc


@pytest.mark.parametrize("order", ["experts_first", "dispatcher_first"])
def test_convert_replaces_configs_in_either_order(order):
    mc = _model(score_before=False, K=2)
    ge = pkg.HipGroupedExpertsConverter(pkg.HipGroupedExpertsConverter.Config(swiglu_limit=7.0))
    td = pkg.HipTokenDispatcherConverter(pkg.HipTokenDispatcherConverter.Config())
    convs = [ge, td] if order == "experts_first" else [td, ge]
    for c in convs:
        c.convert(mc)
    for cfg in (mc.layers[0], mc.layers[1], mc.block.moe):
        assert isinstance(cfg, pkg.HipGroupedExperts.Config)
        assert cfg.swiglu_limit == 7.0
        assert isinstance(cfg.token_dispatcher, pkg.HipTokenDispatcher.Config)
        assert cfg.token_dispatcher.top_k == 2
    assert mc.layers[0].token_dispatcher.score_before_experts is False
    assert mc.layers[0].dim == 256 and mc.block.moe.dim == 128


def test_build_converted_module():
    mc = _model()
    pkg.HipGroupedExpertsConverter(pkg.HipGroupedExpertsConverter.Config()).convert(mc)
    pkg.HipTokenDispatcherConverter(pkg.HipTokenDispatcherConverter.Config()).convert(mc)
    m = mc.layers[0].build()
    assert isinstance(m, pkg.HipGroupedExperts)
    assert isinstance(m.token_dispatcher, pkg.HipTokenDispatcher)
    assert m.w13.shape == (8, 1024, 256) and m.w2.shape == (8, 256, 512)
    m._init_self_parameters()
    assert 0.015 < m.w13.std().item() < 0.025
    assert m.token_dispatcher.is_local


def test_unconverted_dispatcher_is_not_silently_replaced():
    mc = _model()
    pkg.HipGroupedExpertsConverter(pkg.HipGroupedExpertsConverter.Config()).convert(mc)
    m = mc.layers[0].build()
    assert not isinstance(m.token_dispatcher, pkg.HipTokenDispatcher)
    with pytest.raises(NotImplementedError):
        m(torch.zeros(1, 2, 256), torch.ones(2, 1), torch.zeros(2, 1, dtype=torch.int64))


def test_cpu_tensors_have_no_fallback():
    m = pkg.HipGroupedExperts.Config(
        dim=256, hidden_dim=128, num_experts=4,
        token_dispatcher=pkg.HipTokenDispatcher.Config(num_experts=4, top_k=1),
    ).build()
    with pytest.raises(RuntimeError, match="HIP device"):
        m(torch.zeros(1, 4, 256), torch.ones(4, 1), torch.zeros(4, 1, dtype=torch.int64))


def test_import_has_no_side_effects():
    # importing the package patches nothing in torch (the reference's
    # `import torchtitanturbo` monkeypatches at import, patch.py:31-50)
    import subprocess
    import sys

    code = (
        "import importlib, torch, torch.nn.functional as F\n"
        "before = (torch._grouped_mm, F.silu, torch.argsort)\n"
        "importlib.import_module('torchtitan-ascend_amd')\n"
        "assert before == (torch._grouped_mm, F.silu, torch.argsort)\n"
    )
    from conftest import ROOT

    subprocess.run([sys.executable, "-c", code], check=True, cwd=ROOT)


class _FakeMesh:
    def __init__(self, n):
        self.n = n

    def size(self):
        return self.n


def _dispatcher(**cfg):
    return pkg.HipTokenDispatcher.Config(num_experts=4, top_k=1, **cfg).build()


def test_is_local_needs_a_provable_expert_parallel_degree(monkeypatch):
    """The single-GPU path is taken only when the expert-parallel degree is
    provably 1; several torch.distributed ranks with nothing saying how the
    experts are shared is an error, not a silent local run on a shard."""
    d = _dispatcher()
    assert d.is_local  # no process group at all
    import torch.distributed as dist

    monkeypatch.setattr(dist, "is_initialized", lambda: True)
    monkeypatch.setattr(dist, "get_world_size", lambda *a, **k: 8)
    with pytest.raises(RuntimeError, match="expert_parallel_degree"):
        _ = d.is_local
    with pytest.raises(RuntimeError, match="expert_parallel_degree"):
        d.dispatch(torch.zeros(2, 256), torch.ones(2, 1), torch.zeros(2, 1, dtype=torch.int64))
    # declared: data parallelism only, or a real expert-parallel degree
    assert _dispatcher(expert_parallel_degree=1).is_local
    d4 = _dispatcher(expert_parallel_degree=4)
    assert not d4.is_local
    with pytest.raises(NotImplementedError, match="expert-parallel"):
        d4.dispatch(torch.zeros(2, 256), torch.ones(2, 1), torch.zeros(2, 1, dtype=torch.int64))
    # an attached mesh decides, whatever its attribute name
    for name in ("ep_mesh", "device_mesh", "process_group"):
        d1 = _dispatcher()
        setattr(d1, name, _FakeMesh(1))
        assert d1.is_local
        d2 = _dispatcher(expert_parallel_degree=1)
        setattr(d2, name, _FakeMesh(2))
        assert not d2.is_local


def test_dispatcher_converter_passes_the_degree():
    mc = _model()
    pkg.HipTokenDispatcherConverter(pkg.HipTokenDispatcherConverter.Config(expert_parallel_degree=1)).convert(mc)
    assert mc.layers[0].token_dispatcher.expert_parallel_degree == 1


def test_expert_tp_degree_from_dtensor_placements(tmp_path, monkeypatch):
    """w2 sharded on its hidden dim (Shard(2), npu_gmm.py:79-83) over a mesh
    of one rank holds the whole weight and runs as is; a degree above one
    needs the reference's all-reduce and raises instead of returning a
    partial sum."""
    import torch.distributed as dist
    from torch.distributed.device_mesh import init_device_mesh
    from torch.distributed.tensor import Replicate, Shard, distribute_tensor

    GE = importlib.import_module("torchtitan-ascend_amd.grouped_experts")
    dist.init_process_group("gloo", init_method=f"file://{tmp_path}/pg", rank=0, world_size=1)
    try:
        mesh = init_device_mesh("cpu", (1,))
        w = torch.randn(4, 16, 8)
        local, tp = GE._local(distribute_tensor(w, mesh, [Shard(2)]))
        assert tp == 1 and torch.equal(local, w)
        assert GE._local(distribute_tensor(w, mesh, [Replicate()]))[1] == 1
        assert GE._local(w)[1] == 1
    finally:
        dist.destroy_process_group()
    m = pkg.HipGroupedExperts.Config(
        dim=256, hidden_dim=128, num_experts=4,
        token_dispatcher=pkg.HipTokenDispatcher.Config(num_experts=4, top_k=1),
    ).build()
    monkeypatch.setattr(GE, "_local", lambda p: (p, 2))
    with pytest.raises(NotImplementedError, match="degree 2"):
        m._weights()

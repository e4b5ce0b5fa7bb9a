"""The names the reference's callers of the MoE layer import resolve in this package, so those files
run unchanged: transformer_block.py:11-15, transformer_moe.py:11-14, tests/test_moe.py:3-5,
tests/test_moe_ep.py:9-11 and examples/train_gpt_moe.py:14-18.  Also MLPTensorParallel's
one-process behaviour (mlp.py:41-81)."""

import importlib

import pytest
import torch

IMPORTS = {
    # transformer_block.py:11-15
    "abacus.attention": ["MultiHeadAttention"],
    "abacus.distributed.expert_parallel": ["_rank_and_world_size"],
    "abacus.mlp": ["MLP", "MLPTensorParallel"],
    "abacus.moe.moe": ["MoE", "MoEExpertParallel"],
    "abacus.norm": ["RMSNorm"],
    # transformer_moe.py:11-14
    "abacus.embedding": ["Embedding"],
    "abacus.rope": ["Rotary"],
    "abacus.transformer_block": ["TransformerBlockMoe"],
    # tests/test_moe.py:3-5, tests/test_moe_ep.py:9-11
    "abacus.moe.router": ["Router"],
    "abacus.transformer_moe": ["TransformerMoe"],
    # examples/train_gpt_moe.py:14-18
    "abacus.distributed.utils": ["init_process_group", "dist_env_vars", "rank", "shutdown", "world_size"],
    "abacus.kernels.liger": ["set_use_liger"],
    "abacus.model_config": ["DIM", "HEAD_DIM", "N_BLOCKS", "N_HEADS"],
    "abacus.trainer": ["Trainer", "get_device"],
}


@pytest.mark.parametrize("module", sorted(IMPORTS))
def test_caller_imports_resolve(module):
    mod = importlib.import_module(module)
    for name in IMPORTS[module]:
        assert hasattr(mod, name), f"{module}.{name}"


def test_mlp_tensor_parallel_one_process_equals_mlp():
    """One process: the same parameters, shapes and seeded values as MLP, and the same output."""
    from abacus.mlp import MLP, MLPTensorParallel

    torch.manual_seed(0)
    dense = MLP(24, 40)
    torch.manual_seed(0)
    tp = MLPTensorParallel(24, 40, sequence_parallel=True)
    assert (tp.rank, tp.world_size, tp.sequence_parallel) == (0, 1, True)
    assert list(tp.state_dict()) == ["w_gate_DM", "w_up_DM", "w_down_MD"]
    for name, p in dense.state_dict().items():
        assert torch.equal(tp.state_dict()[name], p), name
    x = torch.randn(2, 5, 24)
    assert torch.equal(tp(x), dense(x))
    assert MLPTensorParallel(16).hidden_dim == 16


def test_mlp_tensor_parallel_refuses_several_processes(monkeypatch):
    import abacus.mlp as mlp

    monkeypatch.setattr(mlp, "_rank_and_world_size", lambda: (1, 4))
    with pytest.raises(NotImplementedError, match="4 processes"):
        mlp.MLPTensorParallel(32, 64)

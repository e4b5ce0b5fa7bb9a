"""The caller path of examples/train_gpt_moe.py on this build.

The example imports (examples/train_gpt_moe.py:12-16) resolve to this package, and its
single-process flow -- documents from a {"tokens": [1-D LongTensor], "vocab_size": int} file
(:26-33), documents under 2 tokens dropped and --limit applied (:36-49), batches of 4 padded
with -100 (:52-65), seed 0, TransformerMoe(DIM, N_HEADS, HEAD_DIM, N_BLOCKS, vocab, E=4, K=1)
and Trainer(model, total_steps) stepping over the batches (:91-134) -- trains on one GPU, and on
the CPU (the MoE layers on the host build of the library): the loss is finite and falls, and
every router's selection bias moves (router.py:52-53).  The data
file is synthetic (Zipf-distributed token ids), written by the test; the reference's data
comes from a network-bound prep script.
"""

from __future__ import annotations

import os
import sys

import pytest
import torch

from abacus.distributed.utils import dist_env_vars, init_process_group, rank, shutdown, world_size
from abacus.kernels.liger import set_use_liger
from abacus.model_config import DIM, HEAD_DIM, N_BLOCKS, N_HEADS
from abacus.trainer import Trainer, get_device
from abacus.transformer_moe import TransformerMoe

N_EXPERTS, TOP_K, BATCH_SIZE = 4, 1, 4  # examples/train_gpt_moe.py:22-24


def _write_documents(path, n_docs=40, vocab=512, seed=0):
    gen = torch.Generator().manual_seed(seed)
    p = 1.0 / torch.arange(1, vocab + 1, dtype=torch.float64) ** 1.1
    docs = []
    for i in range(n_docs):
        length = int(torch.randint(1, 97, (1,), generator=gen))  # some documents are too short to keep
        docs.append(torch.multinomial(p, length, replacement=True, generator=gen).to(torch.long))
    torch.save({"tokens": docs, "vocab_size": vocab}, path)
    return docs


def _batches(docs, batch_size):
    usable = len(docs) // batch_size * batch_size
    for start in range(0, usable, batch_size):
        group = docs[start:start + batch_size]
        out = torch.full((batch_size, max(d.numel() for d in group)), -100, dtype=torch.long)
        for row, d in enumerate(group):
            out[row, :d.numel()] = d
        yield out


def _run_example(path, limit):
    """The example's single-process main() body on this package."""
    device = get_device()
    set_use_liger(False)
    assert not dist_env_vars()
    saved = torch.load(path, weights_only=True)
    docs = [d for d in saved["tokens"][:limit] if d.numel() >= 2]
    vocab = int(saved["vocab_size"])
    total_steps = len(docs) // BATCH_SIZE
    torch.manual_seed(0)
    model = TransformerMoe(dim=DIM, n_heads=N_HEADS, head_dim=HEAD_DIM, n_blocks=N_BLOCKS, vocab_size=vocab,
                           n_experts=N_EXPERTS, top_k=TOP_K, expert_parallel=False).to(device)
    bias0 = [b.moe.router.expert_bias_E.detach().clone() for b in model.blocks]
    trainer = Trainer(model, total_steps=total_steps)
    losses = []
    for tokens_BL in _batches(docs, BATCH_SIZE):
        loss, _ = trainer.step(tokens_BL.to(device))
        losses.append(float(loss))
    moved = [not torch.equal(b0, b.moe.router.expert_bias_E.detach()) for b0, b in zip(bias0, model.blocks)]
    return losses, moved, total_steps


def _check_training(tmp_path):
    path = tmp_path / "docs.pt"
    _write_documents(path)
    losses, moved, total_steps = _run_example(path, limit=40)
    print(f"[example] {total_steps} steps, losses {[round(v, 3) for v in losses]}", flush=True)
    assert len(losses) == total_steps >= 6
    assert all(torch.isfinite(torch.tensor(losses)))
    assert sum(losses[-2:]) < sum(losses[:2])
    assert all(moved)


@pytest.mark.gpu
def test_example_trains_on_one_gpu(tmp_path):
    _check_training(tmp_path)


def test_example_trains_on_cpu(tmp_path, monkeypatch):
    import abacus_amd.train as train
    monkeypatch.setattr(train, "get_device", lambda: torch.device("cpu"))
    monkeypatch.setattr(sys.modules[__name__], "get_device", lambda: torch.device("cpu"))
    _check_training(tmp_path)


def test_process_group_helpers_single_process(monkeypatch):
    """init_process_group / rank / world_size / shutdown (distributed/utils.py:9-33) as a one-rank
    gloo group over the loopback interface.  Without a group they raise, as torch.distributed's
    get_rank / get_world_size do in the reference."""
    for fn in (rank, world_size):
        with pytest.raises((ValueError, RuntimeError)):
            fn()
    monkeypatch.setenv("RANK", "0")
    monkeypatch.setenv("WORLD_SIZE", "1")
    monkeypatch.setenv("MASTER_ADDR", "127.0.0.1")
    monkeypatch.setenv("MASTER_PORT", str(29500 + os.getpid() % 1000))
    assert dist_env_vars()
    threads = torch.get_num_threads()
    try:
        init_process_group("gloo")
        assert torch.get_num_threads() == 1
        assert (rank(), world_size()) == (0, 1)
    finally:
        shutdown()
        torch.set_num_threads(threads)
    with pytest.raises((ValueError, RuntimeError)):
        rank()

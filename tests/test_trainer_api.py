"""The reference's training entry points on the CPU: WSD (optimizers/lr_scheduler.py),
cross_entropy / set_use_liger (kernels/liger.py) and Trainer's constructor checks
(trainer.py:29-56)."""

import math

import pytest
import torch
import torch.nn.functional as F

from abacus.kernels.liger import cross_entropy, set_use_liger
from abacus.optimizers.lr_scheduler import WSD
from abacus.trainer import Trainer


def test_wsd_schedule_closed_form():
    s = WSD(1000, lr=5e-4)
    assert (s.warmup_steps, s.decay_steps) == (20, 100)
    assert math.isclose(s.learning_rate(1), 5e-4 / 20)
    assert math.isclose(s.learning_rate(20), 5e-4)
    assert s.learning_rate(21) == s.learning_rate(900) == 5e-4
    assert math.isclose(s.learning_rate(901), 5e-4 * (1 - 1 / 100))
    assert math.isclose(s.learning_rate(1000), 0.0, abs_tol=1e-15)
    assert [s.step() for _ in range(3)] == [s.learning_rate(k) for k in (1, 2, 3)]
    short = WSD(10)  # no warmup step, one decay step (10 * 10 // 100): the last step's rate is 0
    assert [short.learning_rate(k) for k in range(1, 11)] == [5e-4] * 9 + [0.0]
    with pytest.raises(ValueError, match="total_steps must be at least 1"):
        WSD(0)
    with pytest.raises(ValueError, match="Invalid learning rate"):
        WSD(10, lr=-1.0)
    with pytest.raises(ValueError, match=r"step must be in 1\.\.10"):
        short.learning_rate(11)


def test_cross_entropy_on_cpu_is_torch_and_liger_needs_cuda():
    torch.manual_seed(0)
    x = torch.randn(12, 7, requires_grad=True)
    t = torch.randint(0, 7, (12,))
    t[3] = -100
    torch.testing.assert_close(cross_entropy(x, t), F.cross_entropy(x, t, ignore_index=-100), rtol=0, atol=0)
    torch.testing.assert_close(cross_entropy(x, t, reduction="sum"), F.cross_entropy(x, t, reduction="sum"))
    set_use_liger(True)
    try:
        with pytest.raises(RuntimeError, match="needs a CUDA tensor"):
            cross_entropy(x, t)
    finally:
        set_use_liger(False)


def test_trainer_refuses_multi_process_parallelism():
    model = torch.nn.Linear(4, 4)
    with pytest.raises(ValueError, match="pipeline parallel does not use DataParallel"):
        Trainer(model, parallel=object(), pipeline=object())
    with pytest.raises(NotImplementedError):
        Trainer(model, parallel=object())

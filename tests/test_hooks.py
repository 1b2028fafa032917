"""The trainer and model hooks that arm the fused head and log TRL's metrics, on the CPU: the
guards hand every unsupported call to the original code, the metric formulas, and the entropy
formula against closed forms and a brute-force sum."""

import math
import types

import pytest
import torch

from hackathon_amd import cross_entropy, fused_ce

from _trainer_stub import StubSFTTrainer, make_trainer


def test_entropy_from_logits_closed_forms():
    V = 37
    uniform = torch.zeros(3, V)
    torch.testing.assert_close(cross_entropy.entropy_from_logits(uniform),
                               torch.full((3,), math.log(V)))
    peaked = torch.full((2, V), -1e4)
    peaked[:, 5] = 0.0
    torch.testing.assert_close(cross_entropy.entropy_from_logits(peaked), torch.zeros(2))
    g = torch.Generator().manual_seed(0)
    x = torch.randn(300, V, generator=g, dtype=torch.float64)
    p = torch.softmax(x, -1)
    want = torch.tensor([-sum(float(pi) * math.log(float(pi)) for pi in row) for row in p],
                        dtype=torch.float64)
    torch.testing.assert_close(cross_entropy.entropy_from_logits(x, chunk_size=7), want)


def _step(entropy, correct, labelled):
    return types.SimpleNamespace(token_entropy=entropy, correct=torch.tensor(correct),
                                 labelled=torch.tensor(labelled))


def test_log_metrics_formulas():
    t = make_trainer(torch.nn.Linear(2, 2))
    mask = torch.tensor([[1, 1, 1, 0], [1, 1, 0, 0]])
    ent = torch.tensor([[1.0, 2.0, 3.0, 100.0], [4.0, 5.0, 100.0, 100.0]])
    cross_entropy._log_metrics(t, "train", {"attention_mask": mask}, _step(ent, 3, 4))
    assert t._metrics["train"]["entropy"] == [pytest.approx(15.0 / 5.0)]
    assert t._metrics["train"]["num_tokens"] == [5]
    assert t._metrics["train"]["mean_token_accuracy"] == [pytest.approx(0.75)]
    cross_entropy._log_metrics(t, "train", {"attention_mask": mask}, _step(ent, 0, 0))
    assert t._metrics["train"]["num_tokens"] == [10]
    assert t._metrics["train"]["mean_token_accuracy"][-1] == 0.0


def test_trainer_hooks_fall_back_on_cpu():
    """On CPU tensors both hooks hand the call to the trainer's own compute_loss."""
    calls = []

    class Orig(StubSFTTrainer):
        def compute_loss(self, model, inputs, return_outputs=False, num_items_in_batch=None):
            calls.append(inputs)
            return torch.tensor(1.5)

    class A(Orig):
        pass

    class B(Orig):
        pass

    assert cross_entropy._patch_trainer(A)
    model = torch.nn.Linear(2, 2).train()
    inputs = {"labels": torch.zeros(1, 3, dtype=torch.long),
              "attention_mask": torch.ones(1, 3, dtype=torch.long)}
    assert float(A.compute_loss(make_trainer(model, A), model, dict(inputs))) == 1.5
    assert fused_ce.patch_sft_trainer(B)
    try:
        assert float(B.compute_loss(make_trainer(model, B), model, dict(inputs))) == 1.5
    finally:
        fused_ce.unpatch()
    assert len(calls) == 2
    assert not cross_entropy._can_fuse(make_trainer(model, A), model, inputs)
    assert not fused_ce._can_fuse(make_trainer(model, B), model, inputs)


@pytest.mark.parametrize("change", ["liger", "loss_type", "smoother", "loss_func", "eval",
                                    "no_mask", "shift_labels", "no_metrics"])
def test_can_fuse_guards(change):
    """Every condition of _can_fuse is checked before the device check, on a model that would
    otherwise pass everything except being on a GPU."""
    model = torch.nn.Linear(2, 2).train()
    t = make_trainer(model)
    inputs = {"labels": torch.zeros(1, 3, dtype=torch.long),
              "attention_mask": torch.ones(1, 3, dtype=torch.long)}
    if change == "liger":
        t.args.use_liger_kernel = True
    elif change == "loss_type":
        t.args.loss_type = "dft"
    elif change == "smoother":
        t.label_smoother = object()
    elif change == "loss_func":
        t.compute_loss_func = lambda *a, **k: 0
    elif change == "eval":
        model.eval()
    elif change == "no_mask":
        inputs.pop("attention_mask")
    elif change == "shift_labels":
        inputs["shift_labels"] = inputs["labels"]
    elif change == "no_metrics":
        del t._metrics
    assert not cross_entropy._can_fuse(t, model, inputs)
    assert not fused_ce._can_fuse(t, model, inputs)

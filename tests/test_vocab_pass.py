"""Host logic of the fused lm_head + CE engine on the CPU: how rows are grouped under the
logits budget, and the refusal of matmul dtypes the kernels do not take."""

import pytest
import torch

from hackathon_amd import cross_entropy, vocab_pass


@pytest.mark.parametrize("n,vocab,chunk", [(8192, 151936, 512), (4096, 152064, 512),
                                           (10000, 151936, 512), (3, 1000, 512),
                                           (70000, 151936, 512), (2049, 4096, 7), (0, 10, 4)])
def test_groups_cover_rows_within_budget(n, vocab, chunk):
    groups = vocab_pass.plan_groups(n, vocab, chunk)
    covered = [r for a, b in groups for r in range(a, b)]
    assert covered == list(range(n))  # in order, each row once
    cap = chunk * max(1, vocab_pass.LOGITS_BUDGET // (chunk * vocab * 2))
    assert all(b - a <= cap for a, b in groups)
    if groups:
        # as few groups as the budget allows, all of one size but the last
        assert len(groups) == -(-n // cap)
        assert len({b - a for a, b in groups[:-1]}) <= 1
        assert groups[-1][1] - groups[-1][0] <= groups[0][1] - groups[0][0]


def test_qwen_shapes_group_sizes():
    # 8192 x 151936 (2.49 GB of bf16 logits) never lives whole: two groups of 4096 rows; the 7B
    # step's 4096 x 152064 (1.25 GB) is one group
    assert vocab_pass.plan_groups(8192, 151936, 512) == [(0, 4096), (4096, 8192)]
    assert vocab_pass.plan_groups(4096, 152064, 512) == [(0, 4096)]
    # a budget of one chunk gives the reference's 512-row chunks
    assert vocab_pass.plan_groups(2000, 151936, 512, budget=1) == \
        [(0, 512), (512, 1024), (1024, 1536), (1536, 2000)]


def test_fp32_matmul_dtype_is_refused_before_any_launch():
    h = torch.randn(4, 8)
    w = torch.randn(16, 8)
    t = torch.zeros(4, dtype=torch.long)
    with pytest.raises(TypeError, match="fp16 or bf16"):
        cross_entropy.FusedLinearCrossEntropy.apply(h, w, t, torch.tensor(4), torch.float32, 512)
    with pytest.raises(TypeError, match="fp16 or bf16"):
        cross_entropy.fused_causal_lm_loss(h[None], w, t[None])


def test_fp32_model_keeps_its_own_forward():
    """A Qwen2 causal LM whose head matmul would run in fp32 is not taken by the model hook
    (the kernels are 16-bit); in bf16, or under autocast, it is (head checks aside)."""
    from types import SimpleNamespace

    lm = SimpleNamespace(
        lm_head=torch.nn.Linear(8, 16, bias=False).requires_grad_(False),
        config=SimpleNamespace(final_logit_softcapping=None),
        model=SimpleNamespace(norm=SimpleNamespace(weight=torch.ones(8)),
                              embed_tokens=SimpleNamespace(weight=torch.ones(16, 8))))
    assert cross_entropy._matmul_dtype(torch.float32, torch.float32) == torch.float32
    dt = cross_entropy._matmul_dtype(cross_entropy._hidden_dtype(lm), lm.lm_head.weight.dtype)
    assert dt not in cross_entropy.MATMUL_DTYPES
    assert not cross_entropy._head_ok(lm)  # on the CPU it is refused for the device as well


def test_explicit_chunk_rows_bound_the_live_logits():
    """The default chunk argument lets groups grow to the engine's budget; an explicitly passed
    chunk size (a plain int, 512 included) bounds every group at that many rows, as the
    reference's chunk loop does."""
    import inspect

    from hackathon_amd import fused_ce

    default = inspect.signature(cross_entropy.fused_causal_lm_loss).parameters["chunk_rows"].default
    assert default == 512 and repr(default) == "512"
    assert vocab_pass.budget_for(default) == vocab_pass.LOGITS_BUDGET
    assert vocab_pass.budget_for(fused_ce.CHUNK) == vocab_pass.LOGITS_BUDGET
    for chunk in (512, 256, 1000):
        groups = vocab_pass.plan_groups(8192, 151936, chunk, 2, vocab_pass.budget_for(chunk))
        assert max(b - a for a, b in groups) <= chunk
        assert [r for a, b in groups for r in range(a, b)] == list(range(8192))
    groups = vocab_pass.plan_groups(8192, 151936, default, 2, vocab_pass.budget_for(default))
    assert groups == [(0, 4096), (4096, 8192)]

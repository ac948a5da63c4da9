"""The SmolLM-135M-shaped LoRA training step captured in a HIP graph
(train_bench.capture_step) against the same step run eagerly, and the
no-wait LM-head loss (cfops_lm_head_ce_dev) against the waiting one.

Every replay, with the program's own eager work and synchronizations between
replays, must give the eager step's loss and gradients bit for bit: the
captured kernels are the eager ones in the same order, and none of them uses
atomics.
"""
import pytest
import torch

from cpuforge_amd import ops as P
from cpuforge_amd._lib import CfattnError
from cpuforge_amd.train_bench import SmolLM, capture_step

pytestmark = pytest.mark.gpu


def test_graph_replays_match_the_eager_step():
    B, S, vocab = 2, 128, 4096
    model = SmolLM(layers=2, seq=S, rank=16, dtype=torch.float32, device="cuda", backend="cfops",
                   config={"vocab": vocab})
    gen = torch.Generator(device="cuda")
    gen.manual_seed(3)
    tokens = torch.randint(0, vocab, (B, S), generator=gen, device="cuda")
    targets = torch.randint(0, vocab, (B, S), generator=gen, device="cuda")
    targets[0, :5] = P.IGNORE_INDEX
    params = model.params()
    for p in params:
        p.grad = None
    loss = model.loss(tokens, targets)
    loss.backward()
    ref_loss = loss.item()
    ref = [p.grad.clone() for p in params]
    del loss

    model.ce_on_device = True
    graph, static_loss = capture_step(model, tokens, targets)
    for rep in range(3):
        print(f"replay {rep}", flush=True)
        graph.replay()
        torch.cuda.synchronize()
        model.check_targets()
        assert static_loss.item() == ref_loss, rep
        for i, (p, r) in enumerate(zip(params, ref)):
            assert torch.equal(p.grad, r), (rep, i)
        # The program's own eager work between replays.
        x = torch.randn(256, 256, device="cuda")
        (x @ x).sum().item()
        torch.cuda.synchronize()


def test_device_loss_matches_the_host_loss_and_reports_a_bad_target():
    t, d, vocab = 8, 64, 5
    gen = torch.Generator(device="cuda")
    gen.manual_seed(5)
    hn = torch.randn(t, d, device="cuda", generator=gen)
    head = torch.randn(vocab, d, device="cuda", generator=gen)
    targets = torch.tensor([0, 1, 2, 3, 4, 5, 1, P.IGNORE_INDEX], device="cuda")
    dhn = torch.empty_like(hn)
    res = P.ce_result_buffer("cuda")
    with pytest.raises(CfattnError, match="target 5 out of range for vocab 5"):
        P.lm_head_ce(hn, head, targets, t, d, vocab, dhn)
    P.lm_head_ce_dev(hn, head, targets, t, d, vocab, dhn, None, res)
    with pytest.raises(CfattnError, match="target 5 out of range for vocab 5"):
        P.ce_check(res, targets, vocab)

    targets[5] = 0
    dhn2 = torch.empty_like(hn)
    dhead, dhead2 = torch.zeros_like(head), torch.zeros_like(head)
    host = P.lm_head_ce(hn, head, targets, t, d, vocab, dhn, dhead)
    P.lm_head_ce_dev(hn, head, targets, t, d, vocab, dhn2, dhead2, res)
    P.ce_check(res, targets, vocab)
    assert P.ce_result_loss(res).item() == host
    assert int(res[0].item()) == t - 1  # the ignored row is not scored
    assert torch.equal(dhn, dhn2) and torch.equal(dhead, dhead2)

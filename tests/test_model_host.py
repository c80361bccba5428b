"""CPU: the host-side logic of the model orchestration (testt_amd/model.py) against what
transformers defines for it: the causal-LM target shift of ForCausalLMLoss
(transformers/loss/loss_utils.py), the default rotary tables of Qwen2's rotary embedding, and
the per-row rewind losses of HeadStats (solution/model.py:47-51)."""

import torch

from testt_amd import model


def test_shifted_targets_match_for_causal_lm_loss():
    """With all positions real, the shifted targets are exactly what ForCausalLMLoss scores:
    its loss over logits equals cross-entropy against these targets."""
    from transformers.loss.loss_utils import ForCausalLMLoss

    g = torch.Generator().manual_seed(0)
    b, t, v = 3, 11, 37
    labels = torch.randint(0, v, (b, t), generator=g)
    labels[0, :4] = -100
    labels[2, 7:] = -100
    logits = torch.randn(b, t, v, generator=g)
    pos = torch.arange(b * t)
    tgt = model.shifted_targets(labels, pos)
    ref = ForCausalLMLoss(logits, labels, v, num_items_in_batch=None)
    mine = torch.nn.functional.cross_entropy(logits.reshape(-1, v), tgt, ignore_index=-100)
    assert torch.allclose(mine, ref, rtol=1e-6, atol=0)
    # the last position of each row has no target
    assert bool((tgt.view(b, t)[:, -1] == -100).all())


def test_shifted_targets_on_real_rows_only():
    labels = torch.tensor([[5, 6, 7, 8], [9, 10, -100, -100]])
    mask = torch.tensor([[1, 1, 1, 1], [1, 1, 0, 0]])
    pos = mask.reshape(-1).nonzero().squeeze(1)
    assert model.shifted_targets(labels, pos).tolist() == [6, 7, 8, -100, 10, -100]


def test_rotary_tables_match_qwen2_rotary_embedding():
    from transformers import Qwen2Config
    from transformers.models.qwen2.modeling_qwen2 import Qwen2RotaryEmbedding

    cfg = Qwen2Config(hidden_size=256, num_attention_heads=2, num_key_value_heads=1,
                      rope_theta=1e6)
    rot = Qwen2RotaryEmbedding(cfg)
    seq = 300
    x = torch.zeros(1, seq, 256)
    cos_ref, sin_ref = rot(x, torch.arange(seq)[None])
    cos, sin = model.rotary_tables(rot.inv_freq, seq)
    assert torch.equal(cos, cos_ref[0]) and torch.equal(sin, sin_ref[0])
    assert torch.equal(model.default_inv_freq(128, 1e6, "cpu"), rot.inv_freq)


def test_head_stats_row_losses():
    st = model.HeadStats(entropy_sum=torch.tensor(0.0), correct=torch.tensor(0),
                         labelled=torch.tensor(5), row_loss_sum=torch.tensor([3.0, 0.0, 4.5]),
                         row_tokens=torch.tensor([2, 0, 3]))
    means, tokens = st.row_losses()
    assert tokens == [2, 0, 3]
    assert means == [1.5, 0.0, 1.5]


def test_configure_backward_is_thread_local():
    """configure_backward() (run by testt_amd.apply()) turns off autograd's device worker
    thread for backward passes started from the calling thread only, and gradients are the
    same either way."""
    import threading

    import testt_amd

    seen = {}

    def worker():
        testt_amd.configure_backward()
        seen["worker"] = torch._C._is_multithreading_enabled()
        x = torch.randn(5, 3, generator=torch.Generator().manual_seed(1), requires_grad=True)
        (x.sin() * x).sum().backward()
        seen["grad"] = x.grad.clone()
        testt_amd.configure_backward(single_threaded=False)
        seen["restored"] = torch._C._is_multithreading_enabled()

    before = torch._C._is_multithreading_enabled()
    th = threading.Thread(target=worker)
    th.start()
    th.join()
    assert seen["worker"] is False and seen["restored"] is True
    assert torch._C._is_multithreading_enabled() == before     # this thread is untouched
    x = torch.randn(5, 3, generator=torch.Generator().manual_seed(1), requires_grad=True)
    (x.sin() * x).sum().backward()
    assert torch.equal(x.grad, seen["grad"])

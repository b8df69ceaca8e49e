"""The condU model around the DSQG layers (dwarf_amd/generation.py): state-dict compatibility
with train/train_2048_condU.py:320-365, the reference's sampling rule, and incremental
generation (prefill + one decode step per token) against the reference's full recomputation
(train/train_2048_condU.py:463-487)."""

import pytest
import torch

from dwarf_amd.generation import CondMTransformer, _sample


def _expected_keys(V, E, L, H, F, T, full=5, interval=3, J=44):
    HD = E // H
    keys = {"embedding.weight": (V, E), "pos_embed.weight": (T + 2, E), "norm.weight": (E,),
            "norm.bias": (E,), "out.weight": (V, E)}
    lin = lambda n, o, i: {f"{n}.weight": (o, i), f"{n}.bias": (o,)}
    for i in range(L):
        p = f"blocks.{i}."
        blk = {}
        for n in ("norm1", "norm2"):
            blk.update({f"{n}.weight": (E,), f"{n}.bias": (E,)})
        blk.update(lin("attn.qkv_proj", 3 * E, E))
        blk.update(lin("attn.out_proj", E, E))
        blk.update(lin("attn.gate_proj", E, E))
        blk.update(lin("ffn.fc1", F, E))
        blk.update(lin("ffn.fc2", E, F))
        if i != full:
            blk.update({"attn.pos_bias": (J, H), "attn.scale_embed": (J, HD), "attn.if_gain": (H,)})
            if i % interval == interval - 1:
                blk.update({"inter_norm.weight": (E,), "inter_norm.bias": (E,)})
                for n in ("inter_gate", "inter_k_proj", "inter_v_proj"):
                    blk.update(lin(n, E, E))
        keys.update({p + k: v for k, v in blk.items()})
    return keys


def test_state_dict_matches_reference_layout():
    m = CondMTransformer(1000, 256, 6, 8, 1024, 2048)
    got = {k: tuple(v.shape) for k, v in m.state_dict().items()}
    assert got == _expected_keys(1000, 256, 6, 8, 1024, 2048)
    assert m.out.weight is m.embedding.weight
    assert torch.all(m.blocks[0].attn.gate_proj.bias == 0)
    assert abs(m.embedding.weight.std().item() - 0.02) < 2e-3


def test_sampling_rule():
    logits = torch.tensor([[0.0, 5.0, 1.0, -2.0], [3.0, 0.0, 0.0, 2.9]])
    assert _sample(logits, 0.0, 0.9, None).tolist() == [1, 0]
    g = torch.Generator().manual_seed(0)
    # top_p small: only the most likely token survives the nucleus cut
    for _ in range(20):
        assert _sample(logits, 1.0, 0.05, g).tolist() == [1, 0]
    # top_p = 1: every token is possible
    seen = {int(_sample(logits[1:], 1.0, 1.0, g)) for _ in range(400)}
    assert seen == {0, 1, 2, 3}


def _model(dev, seq_len=256):
    torch.manual_seed(5)
    m = CondMTransformer(512, 256, 6, 8, 512, seq_len, dropout=0.0).to(dev).eval()
    with torch.no_grad():  # move the zero/one inits so every parameter matters
        for b in m.blocks:
            if hasattr(b.attn, "pos_bias"):
                b.attn.pos_bias.add_(0.3 * torch.randn_like(b.attn.pos_bias))
                b.attn.scale_embed.copy_(0.5 * torch.randn_like(b.attn.scale_embed))
                b.attn.if_gain.copy_(0.8 + 0.4 * torch.rand_like(b.attn.if_gain))
    return m


@pytest.mark.gpu
def test_prefill_then_steps_equal_forward_logits(gpu_device):
    """fp32: logits of prefill + decode steps equal the full forward's, position by position."""
    m = _model(gpu_device)
    g = torch.Generator().manual_seed(9)
    ids = torch.randint(0, 512, (2, 120), generator=g).to(gpu_device)
    N0 = 100
    with torch.no_grad():
        full = m(ids)
        caches = m.new_cache(2)
        pre = m.prefill(ids[:, :N0], caches)
        steps = [m.step(ids[:, t], caches) for t in range(N0, 120)]
    scale = full.abs().max().item()
    assert (pre - full[:, :N0]).abs().max().item() <= 1e-4 * scale
    got = torch.stack(steps, dim=1)
    err = (got - full[:, N0:]).abs().max().item()
    assert err <= 1e-4 * scale, f"step logits err {err:.3g} vs scale {scale:.3g}"
    # Past the position table the step refuses on the host, before launching anything.
    small = _model(gpu_device, seq_len=64)
    with torch.no_grad():
        c2 = small.new_cache(1)
        small.prefill(ids[:1, :63], c2)
        small.step(ids[:1, 63], c2)
        with pytest.raises(ValueError):
            small.step(ids[:1, 64], c2)


def _reference_generate(m, ids, max_new):
    """The reference's loop: the whole model on the last seq_len tokens for every token."""
    with torch.no_grad():
        for _ in range(max_new):
            logits = m(ids[:, -m.seq_len:])[:, -1]
            ids = torch.cat([ids, logits.argmax(-1, keepdim=True)], dim=1)
    return ids


@pytest.mark.gpu
@pytest.mark.parametrize("N0,max_new", [(40, 24), (250, 12)])
def test_greedy_generation_matches_full_recompute(gpu_device, N0, max_new):
    """Greedy decoding: incremental generation picks the same tokens as the reference's full
    recomputation, within the position table (40 + 24) and across its end (250 + 12 passes
    seq_len = 256, where both recompute on the sliding window)."""
    m = _model(gpu_device)
    g = torch.Generator().manual_seed(N0)
    ids = torch.randint(0, 512, (2, N0), generator=g).to(gpu_device)
    got = m.generate(ids, max_new, temperature=0.0)
    ref = _reference_generate(m, ids, max_new)
    assert got.shape == (2, N0 + max_new)
    assert torch.equal(got, ref)
    assert torch.equal(m.generate(ids, max_new, temperature=0.0, use_graph=False), ref)


@pytest.mark.gpu
def test_sampled_generation_graph_equals_eager(gpu_device):
    """Nucleus sampling with a seeded generator: the graph-replayed steps give the same tokens
    as eager steps (the graph is replayed for every token after the second)."""
    m = _model(gpu_device)
    ids = torch.randint(0, 512, (3, 30), generator=torch.Generator().manual_seed(2)).to(gpu_device)
    outs = []
    for use_graph in (True, False):
        gen = torch.Generator(device=gpu_device).manual_seed(77)
        outs.append(m.generate(ids, 40, temperature=0.8, top_p=0.9, generator=gen,
                               use_graph=use_graph))
    assert torch.equal(outs[0], outs[1])


@pytest.mark.gpu
def test_bf16_generation_graph_equals_eager(gpu_device):
    """The model in bf16 (DSQG layers on the MFMA kernels, the full-attention layer attended in
    fp32): graph-replayed greedy generation equals eager steps token for token."""
    m = _model(gpu_device).to(torch.bfloat16)
    ids = torch.randint(0, 512, (2, 50), generator=torch.Generator().manual_seed(4)).to(gpu_device)
    a = m.generate(ids, 30, temperature=0.0)
    b = m.generate(ids, 30, temperature=0.0, use_graph=False)
    assert torch.equal(a, b)

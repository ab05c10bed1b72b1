"""The optimizer driven the way the reference's examples drive it (``examples/quickstart.py``:
a tiny randomly initialised GPT-2 from ``transformers``, offline, ``zero_grad`` / ``backward`` /
``step``; ``examples/train_gpt_small.py:214`` clips gradients to norm 1 before each step).  The
model learns a fixed batch: the loss falls, stays finite, and the state is packed 4-bit."""

from __future__ import annotations

import pytest
import torch

import adamw4bit_amd as aw

pytestmark = pytest.mark.gpu


def tiny_gpt2():
    transformers = pytest.importorskip("transformers")
    config = transformers.GPT2Config(vocab_size=128, n_positions=64, n_embd=64, n_layer=2, n_head=4, n_inner=256,
                                     resid_pdrop=0.0, embd_pdrop=0.0, attn_pdrop=0.0, tie_word_embeddings=False,
                                     use_cache=False)
    torch.manual_seed(42)
    return transformers.GPT2LMHeadModel(config).to("cuda")


@pytest.mark.parametrize("recipe,clip", [("ze-eden", None), ("zip-sr", None), ("zip-sr", 1.0)])
def test_tiny_gpt2_learns_a_batch(recipe, clip):
    model = tiny_gpt2()
    cls = aw.ZEEDENAdamW4Bit if recipe == "ze-eden" else aw.ZIPSRAdamW4Bit
    opt = cls(model.parameters(), lr=3e-3, betas=(0.9, 0.95), weight_decay=0.1, quant_rng_seed=0)
    gen = torch.Generator().manual_seed(0)
    batch = torch.randint(0, 128, (4, 32), generator=gen).to("cuda")
    losses = []
    model.train()
    for _ in range(30):
        opt.zero_grad(set_to_none=True)
        loss = model(batch, labels=batch).loss
        loss.backward()
        if clip is not None:
            norm = opt.clip_grad_norm_(clip)
            assert torch.isfinite(norm)
        opt.step()
        losses.append(float(loss.detach()))
    print(f"{recipe} clip={clip}: loss {losses[0]:.3f} -> {losses[-1]:.3f}", flush=True)
    assert all(torch.isfinite(torch.tensor(losses)))
    assert losses[-1] < 0.6 * losses[0]
    packed = sum(int(bool(getattr(v, "packed", False))) for st in opt.state.values() for k, v in st.items()
                 if k.endswith("_quant_state"))
    assert packed >= 2 * 4  # the 4-bit states of the large matrices (wte, wpe, attn, mlp, head)

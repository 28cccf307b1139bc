"""Config 5 in miniature: a decoder stack whose projections are t8.nn.Linear
(t81lib_amd.nn.Linear in eval mode: K1 pack, then K2 for decode steps and K3 for the
prompt) against the same stack with F.linear in float32 over the same trits.

The two differ only in the projections' summation order (both take the same bf16
activations and the same trits), so the logits agree to float32 rounding carried
through two layers and the bf16 residual stream; greedy tokens agree.
"""

from __future__ import annotations

import pytest
import torch

import bench

pytestmark = pytest.mark.gpu

TINY = dict(layers=2, hidden=256, heads=4, kv_heads=2, ffn=512, vocab=512)


def test_decoder_stack_matches_float_reference(gpu):
    sys_stderr = __import__("sys").__stderr__
    sys_stderr.write("[gpu case] decoder stack tiny\n")
    sys_stderr.flush()
    prompt, steps, batch = 40, 6, 3
    kw = dict(max_batch=batch, max_tokens=prompt + steps, seed=5)
    ours = bench.DecoderStack(torch, gpu, **TINY, **kw)
    ref = bench.DecoderStack(torch, gpu, **TINY, reference=True, **kw)
    g = torch.Generator(gpu).manual_seed(6)
    tokens = torch.randint(0, TINY["vocab"], (batch, prompt), generator=g, device=gpu)
    with torch.no_grad():
        lo, lr = ours.forward(tokens, 0), ref.forward(tokens, 0)
        agree = 0
        for i in range(steps):
            scale = lr.abs().max().item()
            assert (lo - lr).abs().max().item() <= 2e-2 * scale + 1e-3, f"step {i}"
            no, nr = lo.argmax(-1, keepdim=True), lr.argmax(-1, keepdim=True)
            agree += int((no == nr).sum())
            lo, lr = ours.forward(nr, prompt + i), ref.forward(nr, prompt + i)
    assert agree >= 0.9 * steps * batch

"""The Hugging Face Mamba-1 patch on the GPU (check_hf_patch.py's gates, on a
random-init local MambaConfig: real checkpoints need the network).

* logits patched vs unpatched (upstream's torch recurrence) within
  1e-4 * max(1, scale) (check_hf_patch.py:34,67-69);
* engagement: one fast call per layer per forward, no fallbacks;
* cached prefill seeds the recurrent state, and greedy decoding continues
  token-identically (check_hf_patch.py:76-101).
"""

import pytest

from util import case

pytestmark = pytest.mark.gpu


def _model(layers=3, hidden=64, vocab=512, seed=0):
    import torch
    from transformers import MambaConfig, MambaForCausalLM

    cfg = MambaConfig(vocab_size=vocab, hidden_size=hidden, state_size=16,
                      num_hidden_layers=layers, expand=2, conv_kernel=4, time_step_rank=8)
    torch.manual_seed(seed)
    return MambaForCausalLM(cfg).cuda().float().eval()


@pytest.mark.parametrize("conv", [False, True], ids=["scan", "scan+conv"])
@pytest.mark.parametrize("length", [300, 301])
def test_patch_logits_and_engagement(length, conv):
    """300: the gate read in place and the output written time-major; 301 (not a
    multiple of 4): the contiguous scan, then the time-major layout. The default
    patch is the reference's (the scan only); conv=True adds the causal conv."""
    import torch

    import armhackathon_amd as arm_scan

    case(f"hf patch logits L={length} conv={conv}")
    model = _model()
    ids = torch.randint(0, 512, (2, length), device="cuda",
                        generator=torch.Generator(device="cuda").manual_seed(1))
    with torch.no_grad():
        ref = model(ids, use_cache=False).logits
        arm_scan.patch(conv=conv)
        try:
            s0 = arm_scan.stats()
            got = model(ids, use_cache=False).logits
            s1 = arm_scan.stats()
        finally:
            arm_scan.unpatch()
    assert s1["fast_calls"] - s0["fast_calls"] == 3
    assert s1["fallback_calls"] == s0["fallback_calls"]
    assert s1["conv_calls"] - s0["conv_calls"] == (3 if conv else 0)
    assert s1["conv_fallback_calls"] == s0["conv_fallback_calls"]
    scale = max(1.0, ref.abs().max().item())
    assert (got - ref).abs().max().item() < 1e-4 * scale
    assert not arm_scan.stats()["patched"]


def test_patch_config2_architecture():
    """BASELINE config 2 itself: the Mamba-130M architecture (24 layers, d_model 768,
    d_state 16, dt_rank 48, conv 4, vocab 50280), random init, batch 8 x 2048, the
    scan patched (24 fast calls) against upstream's torch recurrence.

    The reference's logit gate, 1e-4 * max(1, scale) between patched and unpatched
    (check_hf_patch.py:34,67-69), is below this model's own fp32 noise: upstream's
    fp32 forward lies about 4.4e-4 of scale from the same model in float64, and two
    fp32 evaluations that round differently inside the scan differ by about 1.8e-4
    after 24 random-init layers. So the gate here is the float64 model: the patched
    fp32 logits are as close to it as upstream's fp32 logits (within 25%), and
    patched and unpatched differ by less than upstream's own fp32 error."""
    import torch
    from transformers import MambaConfig, MambaForCausalLM

    import armhackathon_amd as arm_scan

    case("hf patch config 2 architecture B8 L2048")
    cfg = MambaConfig(vocab_size=50280, hidden_size=768, state_size=16, num_hidden_layers=24,
                      expand=2, conv_kernel=4, time_step_rank=48)
    torch.manual_seed(0)
    model = MambaForCausalLM(cfg).cuda().float().eval()
    ids = torch.randint(0, 50280, (8, 2048), device="cuda",
                        generator=torch.Generator(device="cuda").manual_seed(0))
    with torch.no_grad():
        ref = model(ids, use_cache=False, logits_to_keep=1).logits.double()
        arm_scan.patch()
        try:
            s0 = arm_scan.stats()
            got = model(ids, use_cache=False, logits_to_keep=1).logits.double()
            s1 = arm_scan.stats()
        finally:
            arm_scan.unpatch()
        ref64 = model.double()(ids, use_cache=False, logits_to_keep=1).logits
    assert s1["fast_calls"] - s0["fast_calls"] == 24
    assert s1["fallback_calls"] == s0["fallback_calls"]
    scale = max(1.0, ref64.abs().max().item())
    err_up = (ref - ref64).abs().max().item() / scale      # upstream fp32 vs float64
    err_ours = (got - ref64).abs().max().item() / scale    # patched fp32 vs float64
    gap = (got - ref).abs().max().item() / scale
    print(f"[case] fp32 error vs float64: upstream {err_up:.2e}, patched {err_ours:.2e}; "
          f"patched vs upstream {gap:.2e}", flush=True)
    assert err_ours <= 1.25 * err_up + 1e-6
    assert gap <= err_up


def test_patch_cached_generation():
    import torch

    import armhackathon_amd as arm_scan

    case("hf patch generate")
    model = _model(seed=2)
    ids = torch.randint(0, 512, (1, 64), device="cuda",
                        generator=torch.Generator(device="cuda").manual_seed(3))
    with torch.no_grad():
        ref = model.generate(ids, max_new_tokens=12, do_sample=False)
        arm_scan.patch(conv=True)
        try:
            got = model.generate(ids, max_new_tokens=12, do_sample=False)
            st = arm_scan.stats()
        finally:
            arm_scan.unpatch()
    assert st["fast_calls"] >= 3  # the prefill went through the kernel
    assert st["step_calls"] >= 3 * 11 and st["step_fallback_calls"] == 0  # and the decode
    assert st["conv_calls"] >= 3 * 12 and st["conv_fallback_calls"] == 0  # prefill + steps
    assert torch.equal(ref, got)

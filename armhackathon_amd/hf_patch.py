"""Drop-in acceleration of Hugging Face transformers Mamba-1 on MI355X.

`patch()` replaces the module-level `mamba_selective_scan` of
transformers.models.mamba.modeling_mamba (the seam the reference patches on
transformers >= 5.5, python/arm_scan/patch.py:119-180) with a wrapper that runs
the scan in the HIP kernel. Projections, the causal conv, gating, weights and
caches stay upstream's; only the recurrence moves.

The wrapper takes the fast path for float32 device tensors with no gradient
required; anything else (host tensors, other dtypes, autograd) goes to the
original function unchanged, exactly as the reference's wrapper falls back on
what its kernel cannot serve (python/arm_scan/patch.py:152-168).

Decode steps (one token) go through `mamba_selective_state_update`, which the
reference leaves to upstream (README.md:320-322). It is patched here as well, with
the same fallback rule: the fast path runs the step as one kernel instead of the
dozen small torch kernels upstream launches per layer and token.

`patch(conv=True)` also routes the mixer's depthwise causal convolution
(`causal_conv1d_fn`, the step before the scan, and its decode step) under the same
rule; the default leaves it upstream's, as the reference's patch does. Upstream's
fallback copies the mixer's time-major projection contiguous, runs a depthwise conv
and then a silu pass; the kernel reads the view in place and fuses the bias and the
silu.

The mixer hands the gate z as a (batch, dim, len) view of its time-major
in_proj output and transposes the scan output back for out_proj. The wrapper
reads z in place and writes the output time-major (returned as a (batch, dim,
len) view), so neither side copies; the reference's op copies z
(python/arm_scan/op.py:19-20).

`unpatch()` restores the original; `stats()` reports engagement.
"""

import torch

from .op import (causal_conv1d, causal_conv1d_update, kernel_calls, selective_scan_time_major,
                 selective_state_update)

_STATE = {"orig": None, "orig_step": None, "orig_conv": None, "orig_conv_step": None,
          "target": None,
          "fast_calls": 0, "fallback_calls": 0, "step_calls": 0, "step_fallback_calls": 0,
          "conv_calls": 0, "conv_fallback_calls": 0}


def _patch_conv_fn(modeling_mamba):
    orig = modeling_mamba.causal_conv1d_fn

    def causal_conv1d_fn(hidden_states, weight, bias=None, activation=None, **kwargs):
        tensors = (hidden_states, weight) + (() if bias is None else (bias,))
        needs_grad = torch.is_grad_enabled() and any(t.requires_grad for t in tensors)
        if (needs_grad or activation not in (None, "silu", "swish")
                or any(t.device.type != "cuda" or t.dtype != torch.float32 for t in tensors)
                or hidden_states.dim() != 3 or weight.dim() != 2 or weight.shape[1] > 8):
            _STATE["conv_fallback_calls"] += 1
            return orig(hidden_states, weight, bias=bias, activation=activation, **kwargs)
        _STATE["conv_calls"] += 1
        # the mixer's input is a (b, D, L) view of time-major storage: read in place;
        # the output goes back time-major, so the mixer's x_proj (which reads its
        # transpose) and the scan (which reads it as u, in place) need no copy
        return causal_conv1d(hidden_states, weight, bias=bias, activation=activation,
                             time_major=True)

    modeling_mamba.causal_conv1d_fn = causal_conv1d_fn
    _STATE["orig_conv"] = orig
    if not hasattr(modeling_mamba, "causal_conv1d_update"):
        return
    orig_step = modeling_mamba.causal_conv1d_update

    def causal_conv1d_update_(hidden_states, conv_state, weight, bias=None, activation=None):
        tensors = (hidden_states, conv_state, weight) + (() if bias is None else (bias,))
        needs_grad = torch.is_grad_enabled() and any(t.requires_grad for t in tensors)
        if (needs_grad or activation not in (None, "silu", "swish")
                or any(t.device.type != "cuda" or t.dtype != torch.float32 for t in tensors)
                or hidden_states.dim() != 3 or hidden_states.shape[-1] != 1
                or weight.dim() != 2 or not conv_state.is_contiguous()
                or tuple(conv_state.shape) != (*hidden_states.shape[:2], weight.shape[1])):
            _STATE["conv_fallback_calls"] += 1
            return orig_step(hidden_states, conv_state, weight, bias=bias, activation=activation)
        _STATE["conv_calls"] += 1
        return causal_conv1d_update(hidden_states[..., 0], conv_state, weight, bias=bias,
                                    activation=activation).unsqueeze(-1)

    modeling_mamba.causal_conv1d_update = causal_conv1d_update_
    _STATE["orig_conv_step"] = orig_step


def _patch_step_fn(modeling_mamba):
    orig = modeling_mamba.mamba_selective_state_update

    def mamba_selective_state_update(state, hidden_states, dt, A, B, C, D=None,
                                     dt_bias=None, dt_softplus=False, z=None, **kwargs):
        tensors = (state, hidden_states, dt, A, B, C)
        optional = tuple(t for t in (D, z, dt_bias) if t is not None)
        needs_grad = torch.is_grad_enabled() and any(
            t.requires_grad for t in (*tensors, *optional))
        if (needs_grad or kwargs
                or any(t.device.type != "cuda" for t in (*tensors, *optional))
                or any(t.dtype != torch.float32 for t in (*tensors, *optional))
                or state.dim() != 3 or not state.is_contiguous()):
            _STATE["step_fallback_calls"] += 1
            return orig(state, hidden_states, dt, A, B, C, D=D, dt_bias=dt_bias,
                        dt_softplus=dt_softplus, z=z, **kwargs)
        _STATE["step_calls"] += 1
        return selective_state_update(state, hidden_states, dt, A, B, C, D=D, z=z,
                                      dt_bias=dt_bias, dt_softplus=dt_softplus)

    modeling_mamba.mamba_selective_state_update = mamba_selective_state_update
    _STATE["orig_step"] = orig


def _patch_scan_fn(modeling_mamba, conv):
    orig = modeling_mamba.mamba_selective_scan

    def mamba_selective_scan(hidden_states, dt, A, B, C, D=None, z=None,
                             delta_bias=None, delta_softplus=False,
                             return_last_state=False, use_mambapy=False,
                             use_associative_scan=False, **kwargs):
        tensors = (hidden_states, dt, A, B, C)
        optional = tuple(t for t in (D, z, delta_bias) if t is not None)
        needs_grad = torch.is_grad_enabled() and any(
            t.requires_grad for t in (*tensors, *optional))
        if (needs_grad
                or any(t.device.type != "cuda" for t in (*tensors, *optional))
                or any(t.dtype != torch.float32 for t in tensors)):
            _STATE["fallback_calls"] += 1
            return orig(hidden_states, dt, A, B, C, D=D, z=z, delta_bias=delta_bias,
                        delta_softplus=delta_softplus, return_last_state=return_last_state,
                        use_mambapy=use_mambapy, use_associative_scan=use_associative_scan,
                        **kwargs)
        _STATE["fast_calls"] += 1
        # the mixer's gate is a (b, D, L) view of time-major storage and its out_proj
        # reads scan_output.transpose(1, 2): read z in place and write the output
        # time-major, so neither needs a copy
        return selective_scan_time_major(hidden_states, dt, A, B, C, D=D, z=z,
                                         delta_bias=delta_bias,
                                         delta_softplus=delta_softplus,
                                         return_last_state=return_last_state)

    modeling_mamba.mamba_selective_scan = mamba_selective_scan
    _STATE["orig"] = orig
    _STATE["target"] = "mamba_selective_scan"
    done = ["transformers mamba_selective_scan (selective_scan_fn API)"]
    if hasattr(modeling_mamba, "mamba_selective_state_update"):
        _patch_step_fn(modeling_mamba)
        done.append("transformers mamba_selective_state_update (decode step)")
    if conv and hasattr(modeling_mamba, "causal_conv1d_fn"):
        _patch_conv_fn(modeling_mamba)
        done.append("transformers causal_conv1d_fn (the mixer's causal convolution)")
    return done


def patch(conv=False):
    """Route HF Mamba's selective scan on device tensors through the HIP kernel
    (and its decode step through the single-step kernel), as the reference's
    `patch()` routes the scan (python/arm_scan/patch.py:119-180). With
    `conv=True` the mixer's causal convolution moves to its kernel too.

    Returns the list of patched targets ([] if this transformers version has
    no `mamba_selective_scan` seam). Idempotent: a second call while patched
    changes nothing (unpatch() first to change `conv`).
    """
    if _STATE["orig"] is not None:
        return ["transformers mamba_selective_scan (already patched)"]
    from transformers.models.mamba import modeling_mamba

    if not hasattr(modeling_mamba, "mamba_selective_scan"):
        import warnings

        warnings.warn("armhackathon_amd.patch(): this transformers version has no "
                      "mamba_selective_scan; leaving it unpatched")
        return []
    return _patch_scan_fn(modeling_mamba, conv)


def unpatch():
    """Restore the original implementation (for A/B benchmarking)."""
    if _STATE["orig"] is None:
        return False
    from transformers.models.mamba import modeling_mamba

    modeling_mamba.mamba_selective_scan = _STATE["orig"]
    if _STATE["orig_step"] is not None:
        modeling_mamba.mamba_selective_state_update = _STATE["orig_step"]
    if _STATE["orig_conv"] is not None:
        modeling_mamba.causal_conv1d_fn = _STATE["orig_conv"]
    if _STATE["orig_conv_step"] is not None:
        modeling_mamba.causal_conv1d_update = _STATE["orig_conv_step"]
    _STATE["orig_conv_step"] = None
    _STATE["orig"] = None
    _STATE["orig_step"] = None
    _STATE["orig_conv"] = None
    _STATE["target"] = None
    return True


def stats():
    """Engagement counters: fast-path vs fallback calls, native invocations."""
    return {
        "fast_calls": _STATE["fast_calls"],
        "fallback_calls": _STATE["fallback_calls"],
        "step_calls": _STATE["step_calls"],
        "step_fallback_calls": _STATE["step_fallback_calls"],
        "conv_calls": _STATE["conv_calls"],
        "conv_fallback_calls": _STATE["conv_fallback_calls"],
        "kernel_calls": kernel_calls(),
        "patched": _STATE["orig"] is not None,
        "api": "selective_scan_fn" if _STATE["orig"] is not None else None,
    }

"""Bidirectional selective scan (python/arm_scan/bidirectional.py:98-175).

The same projected tensors traversed in both time directions and merged.
The tied-weights case goes through one call of the bidirectional entry point
(`selective_scan_bidirectional`): where its 16-row blocks fill the chip, both
directions run as two traversals of one launch, each evaluating its own
exp(delta*A) (measured faster than sharing it, whose whole-row scans and barriers
cost more than the exp); rows that fit one on-chip pass on fewer rows take the
kernel that shares exp(delta*A) between the directions; the rest, two launches.
Untied weights (`reverse_params`) run two scans, the backward one in the kernel's
reverse index mode (no flips).

Merge semantics are the reference's: "sum" | "mean" | "concat" | "none"; D and
z apply inside each direction, so a "sum" carries 2*D*u.
"""

import torch

from .op import (selective_scan, selective_scan_bidirectional,
                 selective_scan_bidirectional_with_state)

_MERGES = ("sum", "mean", "concat", "none")


def bidirectional_scan(u, delta, A, B, C, D=None, z=None, delta_bias=None,
                       delta_softplus=False, merge="sum",
                       reverse_params=None, return_last_state=False):
    """Scan `u` forward and backward in time and merge the two outputs.

    Layouts are `selective_scan`'s. `reverse_params` overrides any of "A", "D",
    "delta", "delta_bias", "B", "C" for the backward pass (in forward-time
    layout). With return_last_state=True each output is paired with its final
    state; the backward one is the state after consuming t = 0.
    """
    if merge not in _MERGES:
        raise ValueError(f"merge must be one of {_MERGES}, got {merge!r}")
    if reverse_params is None:
        if return_last_state:
            out_f, out_b, last_f, last_b = selective_scan_bidirectional_with_state(
                u, delta, A, B, C, D=D, z=z, delta_bias=delta_bias,
                delta_softplus=delta_softplus)
        else:
            out_f, out_b = selective_scan_bidirectional(
                u, delta, A, B, C, D=D, z=z, delta_bias=delta_bias,
                delta_softplus=delta_softplus)
    else:
        p = reverse_params
        fwd = selective_scan(u, delta, A, B, C, D=D, z=z, delta_bias=delta_bias,
                             delta_softplus=delta_softplus,
                             return_last_state=return_last_state)
        rev = selective_scan(u, p.get("delta", delta), p.get("A", A), p.get("B", B),
                             p.get("C", C), D=p.get("D", D), z=z,
                             delta_bias=p.get("delta_bias", delta_bias),
                             delta_softplus=delta_softplus,
                             return_last_state=return_last_state, reverse=True)
        if return_last_state:
            (out_f, last_f), (out_b, last_b) = fwd, rev
        else:
            out_f, out_b = fwd, rev

    if merge == "sum":
        out = out_f + out_b
    elif merge == "mean":
        out = (out_f + out_b) * 0.5
    elif merge == "concat":
        out = torch.cat((out_f, out_b), dim=1)
    else:
        out = (out_f, out_b)

    if not return_last_state:
        return out
    return (out, (last_f, last_b)) if merge != "none" else ((out_f, last_f), (out_b, last_b))

"""armhackathon_amd — the MI355X (gfx950) selective-scan engine behind the
`arm_scan` surface of AdityaP9116/ARMHackathon.

The public names are the reference package's (python/arm_scan/__init__.py:24-42):

    import armhackathon_amd as arm_scan
    arm_scan.patch()                       # HF transformers Mamba -> HIP scan
    arm_scan.selective_scan(u, delta, A, B, C, D=..., z=...)
    arm_scan.bidirectional_scan(...)       # both time directions, merged
    arm_scan.ss2d_scan(u, delta, A, B, C)  # four-direction 2D cross-scan
    arm_scan.mamba3_scan(...), mamba3_scan_pair(...), mamba3_mimo_scan(...)
    arm_scan.ss2d_scan_mamba3(...)
    arm_scan.noncausal_scan(...), noncausal_scan_dense(...), ss2d_noncausal_mamba3(...)
    arm_scan.selective_scan_numpy(...)     # numpy in/out (copies through HBM)

Every scan runs in hand-written HIP kernels (libarm_scan_hip.so, built from
armhackathon_amd/csrc/) on PyTorch-ROCm device tensors; there is no CPU path.
"""

from ._ffi import lib_path

__all__ = [
    "lib_path",
    "selective_scan",
    "selective_scan_bidirectional",
    "selective_scan_time_major",
    "selective_state_update",
    "causal_conv1d",
    "causal_conv1d_update",
    "bidirectional_scan",
    "ss2d_scan",
    "use_arm_scan",
    "mamba3_scan",
    "mamba3_scan_pair",
    "mamba3_mimo_scan",
    "ss2d_scan_mamba3",
    "noncausal_scan",
    "noncausal_scan_dense",
    "ss2d_noncausal_mamba3",
    "angles_to_cos_sin",
    "selective_scan_numpy",
    "patch",
    "unpatch",
    "stats",
    "kernel_calls",
]

_LAZY = {
    "selective_scan": ".op",
    "selective_scan_bidirectional": ".op",
    "selective_scan_time_major": ".op",
    "selective_state_update": ".op",
    "causal_conv1d": ".op",
    "causal_conv1d_update": ".op",
    "kernel_calls": ".op",
    "bidirectional_scan": ".bidirectional",
    "ss2d_scan": ".ss2d",
    "use_arm_scan": ".ss2d",
    "mamba3_scan": ".mamba3",
    "mamba3_scan_pair": ".mamba3",
    "mamba3_mimo_scan": ".mamba3",
    "angles_to_cos_sin": ".mamba3",
    "ss2d_scan_mamba3": ".ss2d_mamba3",
    "noncausal_scan": ".mamba3_noncausal",
    "noncausal_scan_dense": ".mamba3_noncausal",
    "ss2d_noncausal_mamba3": ".mamba3_noncausal",
    "selective_scan_numpy": ".numpy_api",
    "patch": ".hf_patch",
    "unpatch": ".hf_patch",
    "stats": ".hf_patch",
}


def __getattr__(name):
    # torch-dependent modules load on first use, as in the reference
    # (python/arm_scan/__init__.py:45-70)
    import importlib

    mod = _LAZY.get(name)
    if mod is None:
        raise AttributeError(f"module 'armhackathon_amd' has no attribute '{name}'")
    return getattr(importlib.import_module(mod, __name__), name)

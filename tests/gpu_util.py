"""Helpers for the GPU parity tests: host <-> device transfer and the parity gate."""
import numpy as np
import torch

# The parity gate against the reference's f32 result: max |a - b| and mean|a - b| / mean|b|.
MAX_ABS = 2e-3
MEAN_REL = 1e-3


def dev(a: np.ndarray, dtype=torch.float32, device="cuda:0") -> torch.Tensor:
    """numpy float32 values (already representable in `dtype`) -> device tensor of `dtype`."""
    t = torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dtype)
    return t.to(device)


def dev_words(w: np.ndarray, device="cuda:0") -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(w, dtype=np.uint32).view(np.int32)).to(device)


def host(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def assert_parity(actual, expected, label="", max_abs=MAX_ABS, mean_rel=MEAN_REL):
    from oracle.oracle import parity_metrics
    m = parity_metrics(actual, expected)
    print(f"[parity] {label} " + " ".join(f"{k}={v:.3e}" if isinstance(v, float) else f"{k}={v}"
                                          for k, v in m.items()), flush=True)
    assert m["finite"], f"{label}: non-finite output"
    assert m["max_abs"] <= max_abs, f"{label}: max_abs {m['max_abs']:.3e} > {max_abs}"
    assert m["mean_rel"] <= mean_rel, f"{label}: mean_rel {m['mean_rel']:.3e} > {mean_rel}"
    return m

"""Helpers shared by the GPU parity tests."""
from __future__ import annotations

import numpy as np
import torch

from maxuna_amd.gguf import ExpertStack, GgmlDType

# tolerance stated by the hot-path contract (fp32 outputs)
REL_L2 = 1e-3
MAX_ABS_OF_RMS = 1e-2


def dev_f32(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()


def dev_u32(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, np.int64)).to(torch.int32).cuda().view(torch.uint32)


def host(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    if t.dtype == torch.uint32:
        return t.view(torch.int32).cpu().numpy().astype(np.uint32)
    return t.cpu().numpy()


def rel_l2(got, want) -> float:
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    return float(np.sqrt(((got - want) ** 2).sum() / max((want ** 2).sum(), 1e-300)))


def assert_close(got, want, rel=REL_L2, max_of_rms=MAX_ABS_OF_RMS, what=""):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    r = rel_l2(got, want)
    rms = float(np.sqrt((want ** 2).mean()))
    mx = float(np.abs(got - want).max()) if got.size else 0.0
    print(f"{what}: rel-L2 {r:.3e}, max-abs/rms {mx / max(rms, 1e-30):.3e}", flush=True)
    assert r <= rel, f"{what}: rel-L2 {r:.3e} > {rel:.1e}"
    assert mx <= max_of_rms * rms + 1e-30, f"{what}: max-abs {mx:.3e} > {max_of_rms:.0e} * rms {rms:.3e}"
    return r, mx


def upload_stack(dtype: GgmlDType, blocks: dict[int, np.ndarray] | np.ndarray, n_expert: int, n_out: int, k: int,
                 base_off: int = 0) -> ExpertStack:
    if isinstance(blocks, dict):
        raw = np.concatenate([blocks[e] for e in range(n_expert)])
    else:
        raw = blocks
    buf = np.zeros(base_off + raw.size, np.uint8)
    buf[base_off:] = raw
    return ExpertStack(torch.from_numpy(buf).cuda(), dtype, n_expert, n_out, k, base_off)


def selection_margin(logits: np.ndarray, bias: np.ndarray, top_k: int) -> np.ndarray:
    """Per token: the smallest gap between adjacent scores among the top_k+1
    largest selection scores (any order decision the top-k makes)."""
    p = (1.0 / (np.exp(-logits.astype(np.float64)) + 1.0))
    sel = np.sort(p + bias, axis=1)[:, ::-1][:, : top_k + 1]
    return np.min(sel[:, :-1] - sel[:, 1:], axis=1)


def check_ids(gpu_ids, orc_ids, margin, eps=1e-5):
    """Expert ids and order must match; a token may differ only if the oracle's
    top-k boundary is a near-tie (margin < eps), which f32 logit rounding can flip."""
    gpu_ids = np.asarray(gpu_ids)
    orc_ids = np.asarray(orc_ids)
    bad = np.nonzero(np.any(gpu_ids != orc_ids, axis=1))[0]
    for r in bad:
        assert margin[r] < eps, f"token {r}: ids {gpu_ids[r].tolist()} vs oracle {orc_ids[r].tolist()} " \
                                f"(boundary margin {margin[r]:.3e})"
    return len(bad)

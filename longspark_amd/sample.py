"""Drafter proposal step on the gfx950 kernel: drop-in for
SRT/speculative/dspark_components/kernels/sample_step_tokens_with_q.py:37-382.

``SRT`` = ``vendor/sglang/python/sglang/srt``.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional, Tuple

import torch

from . import _lib


@dataclass(frozen=True)
class SampleStepWorkspace:
    """Scratch owned by one sequential proposal block (the reference's
    ``_SampleStepWorkspace``, sample_step_tokens_with_q.py:15-29): the noise
    buffer refilled each step and the kernel's counter / tile buffers."""
    batch_size: int
    vocab_size: int
    device: torch.device
    exp_noise: torch.Tensor
    counters: torch.Tensor
    scratch: torch.Tensor
    status: torch.Tensor


def _canonical_cuda_device(device: torch.device) -> torch.device:
    if device.type != "cuda":
        raise ValueError("sample step workspace requires a CUDA device")
    if device.index is None:
        return torch.device("cuda", torch.cuda.current_device())
    return device


def create_sample_step_workspace(*, batch: int, vocab: int, device) -> SampleStepWorkspace:
    """sample_step_tokens_with_q.py:40-69: allocate the scratch of one proposal block."""
    if batch < 0:
        raise ValueError(f"batch must be non-negative, got {batch}")
    if vocab <= 0:
        raise ValueError(f"vocab must be positive, got {vocab}")
    device = _canonical_cuda_device(torch.device(device))
    cb, sb = _lib.workspace_sizes("ls_sample_step_workspace", batch, vocab)
    return SampleStepWorkspace(
        batch_size=batch, vocab_size=vocab, device=device,
        exp_noise=torch.empty((batch, vocab), dtype=torch.float32, device=device),
        counters=torch.zeros(max(cb, 256), dtype=torch.uint8, device=device),
        scratch=torch.empty(max(sb, 256), dtype=torch.uint8, device=device),
        status=torch.zeros(1, dtype=torch.int32, device=device))


def _check_inputs(*, step_logits, temperatures, exp_noise) -> Tuple[int, int]:
    """The input contract of sample_step_tokens_with_q.py:190-221 (same errors)."""
    if step_logits.ndim != 2:
        raise ValueError(f"step_logits must be rank-2, got shape {tuple(step_logits.shape)}")
    if step_logits.dtype not in (torch.float32, torch.bfloat16):
        raise TypeError(f"step_logits must be float32 or bfloat16, got {step_logits.dtype}")
    if not step_logits.is_cuda:
        raise ValueError("sample_step_tokens_with_q requires CUDA step_logits")
    if step_logits.stride(1) != 1:
        raise ValueError("step_logits last dimension must have unit stride")
    n, vocab = step_logits.shape
    if vocab <= 0:
        raise ValueError("step_logits vocabulary dimension must be positive")
    if temperatures.ndim != 1 or temperatures.shape[0] != n:
        raise ValueError(f"temperatures must have shape [{n}], got {tuple(temperatures.shape)}")
    if exp_noise is not None:
        if exp_noise.ndim != 2 or tuple(exp_noise.shape) != (n, vocab):
            raise ValueError(f"exp_noise must have shape [{n}, {vocab}], got {tuple(exp_noise.shape)}")
        if exp_noise.dtype != torch.float32:
            raise TypeError(f"exp_noise must be float32, got {exp_noise.dtype}")
        if not exp_noise.is_cuda:
            raise ValueError("exp_noise must be on CUDA")
        if exp_noise.device != step_logits.device:
            raise ValueError("exp_noise must be on the step_logits device")
    return n, vocab


def _validate_workspace(workspace, *, batch: int, vocab: int, device) -> None:
    if not isinstance(workspace, SampleStepWorkspace):
        raise TypeError("workspace must come from create_sample_step_workspace")
    if workspace.batch_size != batch:
        raise ValueError(f"workspace batch {workspace.batch_size} does not match input batch {batch}")
    if workspace.vocab_size != vocab:
        raise ValueError(f"workspace vocab {workspace.vocab_size} does not match input vocab {vocab}")
    if workspace.device != device:
        raise ValueError(f"workspace device {workspace.device} does not match input device {device}")


def sample_step_tokens_with_q(*, step_logits: torch.Tensor, temperatures: torch.Tensor,
                              exp_noise: Optional[torch.Tensor] = None,
                              workspace: Optional[SampleStepWorkspace] = None,
                              check: bool = False) -> Tuple[torch.Tensor, torch.Tensor]:
    """sample_step_tokens_with_q.py:264-379: per row the exponential race
    ``argmax_v softmax(l / T)_v / E_v`` (E ~ Exp(1); lowest index on ties) and
    that token's probability, in one launch that reads each logit and noise
    value once.  Without ``exp_noise`` the noise is drawn with
    ``exponential_(1)`` as the reference draws it (into the workspace's buffer
    when one is given).

    Invalid rows (NaN or +inf logits, no finite logit, a temperature outside
    (0, inf), noise outside (0, inf) at a finite entry) get token 0 and q = NaN,
    the values the reference stores before its device-side assertion; here
    they are reported without an assertion: ``check=True`` synchronises and
    raises ``RuntimeError``.
    """
    n, vocab = _check_inputs(step_logits=step_logits, temperatures=temperatures, exp_noise=exp_noise)
    device = step_logits.device
    if workspace is not None:
        _validate_workspace(workspace, batch=n, vocab=vocab, device=device)
    if n == 0:
        return (torch.empty((0,), dtype=torch.int64, device=device),
                torch.empty((0,), dtype=torch.float32, device=device))
    temperatures = temperatures.to(device=device, dtype=torch.float32).contiguous()
    if exp_noise is None:
        exp_noise = workspace.exp_noise if workspace is not None else \
            torch.empty((n, vocab), device=device, dtype=torch.float32)
        exp_noise.exponential_(1)
    if exp_noise.stride(1) != 1:
        exp_noise = exp_noise.contiguous()
    next_tokens = torch.empty((n,), dtype=torch.int64, device=device)
    sampled_q = torch.empty((n,), dtype=torch.float32, device=device)
    if workspace is not None:
        cnt, scr, status = workspace.counters, workspace.scratch, workspace.status
    else:
        cnt, scr = _lib.workspaces.get(*_lib.workspace_sizes("ls_sample_step_workspace", n, vocab), device)
        status = torch.zeros(1, dtype=torch.int32, device=device) if check else None
    if check and workspace is not None:
        status.zero_()
    _lib.call("ls_sample_step", step_logits.data_ptr(), _lib.dtype_code(step_logits), step_logits.stride(0), n,
              vocab, temperatures.data_ptr(), exp_noise.data_ptr(), exp_noise.stride(0), next_tokens.data_ptr(),
              sampled_q.data_ptr(), _lib.ptr(status) if check else None, cnt.data_ptr(), cnt.numel(),
              scr.data_ptr(), scr.numel(), _lib.stream_of(device))
    if check:
        torch.cuda.synchronize(device)
        if int(status.item()) != 0:
            raise RuntimeError("sample_step_tokens_with_q: invalid probability row (NaN/+inf logits, no finite "
                               "logit, invalid temperature or noise)")
    return next_tokens, sampled_q


__all__ = ["create_sample_step_workspace", "sample_step_tokens_with_q", "SampleStepWorkspace"]

"""Dense target distributions: drop-ins backed by the gfx950 kernels.

* ``SoftmaxTemp`` / ``softmax_temp`` -- the temperature softmax of
  SPEC/dspark_components/kernels/softmax_temp.py:17-175
  (``ls_softmax_temp``).
* ``build_dflash_verify_target_probs`` -- the dense top-k / top-p target
  distribution of SPEC/dflash_utils.py:743-810 (``ls_target_probs``: the
  verify row scans give each row's support, which is written dense).

``SPEC`` = ``vendor/sglang/python/sglang/srt/speculative``.
"""

from __future__ import annotations

from typing import Any, Optional

import torch

from . import _lib


def _rows(logits: torch.Tensor, what: str) -> torch.Tensor:
    x = logits.reshape(-1, logits.shape[-1]) if logits.dim() != 2 else logits
    if x.stride(-1) != 1:
        x = x.contiguous()
    if x.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        raise ValueError(f"{what}: logits must be fp32, bf16 or fp16 (got {x.dtype})")
    return x


def softmax_temp(*, logits: torch.Tensor, temperatures: torch.Tensor, rows_per_request: int) -> torch.Tensor:
    """``softmax(logits / T)`` per row as fp32 ``[N, V]``; row r uses
    ``temperatures[r // rows_per_request]`` (softmax_temp.py:69-86)."""
    num_rows, vocab = logits.shape[0], logits.shape[-1]
    bs = num_rows // rows_per_request
    assert bs * rows_per_request == num_rows, (
        f"num_rows {num_rows} not divisible by rows_per_request {rows_per_request}")
    what = "softmax_temp"
    dev = _lib.require_cuda(logits, temperatures, what=what)
    x = _rows(logits, what)
    temps = temperatures.reshape(bs).to(device=dev, dtype=torch.float32).contiguous()
    out = torch.empty((num_rows, vocab), dtype=torch.float32, device=dev)
    if num_rows == 0:
        return out
    _lib.call("ls_softmax_temp", x.data_ptr(), _lib.dtype_code(x), x.stride(0), num_rows, vocab, temps.data_ptr(),
              rows_per_request, out.data_ptr(), out.stride(0), _lib.stream_of(dev))
    return out


class SoftmaxTemp:
    """Drop-in for ``SoftmaxTemp`` (softmax_temp.py:17-66): every implementation
    selector runs the gfx950 kernel."""

    @classmethod
    def execute(cls, *args, **kwargs) -> torch.Tensor:
        return cls.hip(*args, **kwargs)

    @classmethod
    def hip(cls, *, logits: torch.Tensor, temperatures: torch.Tensor, rows_per_request: int) -> torch.Tensor:
        return softmax_temp(logits=logits, temperatures=temperatures, rows_per_request=rows_per_request)

    torch = hip
    triton = hip
    flashinfer = hip


def target_probs(*, logits: torch.Tensor, temperatures: torch.Tensor, rows_per_request: int, top_ks=None,
                 top_ps=None, min_ps=None, max_top_k: Optional[int] = None, scan_hint: int = 0,
                 check: bool = False) -> torch.Tensor:
    """Dense fp32 ``[rows, V]`` distribution of each row after temperature,
    top-k (ties at the k-th value to the lowest index), top-p and (optional)
    min-p.  Per-request ``[B]`` parameters; ``top_ks >= V``, ``top_ps >= 1`` and
    ``min_ps <= 0`` (or None) disable a filter.  ``max_top_k``: host upper
    bound of ``top_ks`` (None: no bound known).  With ``check`` the call
    synchronises and raises if a row's support exceeded the kernel's capacity
    (such rows are written as zeros)."""
    what = "target_probs"
    x = _rows(logits, what)
    rows, vocab = x.shape
    if rows_per_request <= 0 or rows % rows_per_request != 0:
        raise ValueError(f"{what}: {rows} rows are not a multiple of rows_per_request {rows_per_request}")
    batch = rows // rows_per_request
    dev = _lib.require_cuda(x, temperatures, what=what)

    def per_request(t, dtype, name):
        if t is None:
            return None
        t = torch.as_tensor(t, device=dev).reshape(-1)
        if t.numel() != batch:
            raise ValueError(f"{what}: {name} must have {batch} entries")
        return t.to(dtype).contiguous()

    temps = per_request(temperatures, torch.float32, "temperatures")
    ks = per_request(top_ks, torch.int32, "top_ks")
    ps = per_request(top_ps, torch.float32, "top_ps")
    mps = per_request(min_ps, torch.float32, "min_ps")
    out = torch.empty((rows, vocab), dtype=torch.float32, device=dev)
    if rows == 0:
        return out
    status = torch.empty(1, dtype=torch.int32, device=dev)  # cleared by the call's first kernel
    mk = 0 if max_top_k is None else int(max_top_k)
    a = _lib.TargetProbsArgs()
    a.logits, a.logits_dtype, a.logits_row_stride = x.data_ptr(), _lib.dtype_code(x), x.stride(0)
    a.batch, a.rows_per_request, a.vocab = batch, rows_per_request, vocab
    a.temperatures, a.top_ks, a.top_ps, a.min_ps = temps.data_ptr(), _lib.ptr(ks), _lib.ptr(ps), _lib.ptr(mps)
    a.max_top_k = mk
    a.out, a.out_row_stride, a.status, a.scan_hint = out.data_ptr(), out.stride(0), status.data_ptr(), scan_hint
    cnt, scr = _lib.workspaces.get(*_lib.workspace_sizes("ls_target_probs_workspace", batch, rows_per_request,
                                                          vocab, mk), dev)
    _lib.call("ls_target_probs", _lib.ctypes.byref(a), cnt.data_ptr(), cnt.numel(), scr.data_ptr(), scr.numel(),
              _lib.stream_of(dev))
    if check:
        torch.cuda.synchronize(dev)
        if int(status.item()) != 0:
            raise RuntimeError(f"{what}: a row's support exceeded the kernel capacity")
    return out


def build_dflash_verify_target_probs(*, next_token_logits: torch.Tensor, sampling_info: Any, draft_token_num: int,
                                     bs: int, max_top_k: Optional[int] = None,
                                     uniform_top_k_value: Optional[int] = None,
                                     use_sparse_topk: bool = True) -> torch.Tensor:
    """Drop-in for SPEC/dflash_utils.py:743-810: ``[bs, draft_token_num, V]``
    fp32 target probabilities.  The sparse top-k-first path keeps
    ``min(top_k, max_top_k)`` entries per row (:761-786); the dense path
    (no sparse top-k, or ``max_top_k >= V``) keeps ``top_k``; top-p applies
    when ``sampling_info.need_top_p_sampling``.  ``uniform_top_k_value`` only
    lets the reference skip a mask and changes no value."""
    ks, ps, mk_bound = dflash_filter_params(sampling_info, int(next_token_logits.shape[-1]), max_top_k,
                                            use_sparse_topk)
    out = target_probs(logits=next_token_logits, temperatures=sampling_info.temperatures,
                       rows_per_request=draft_token_num, top_ks=ks, top_ps=ps, max_top_k=mk_bound)
    return out.view(bs, draft_token_num, -1)


def dflash_filter_params(sampling_info: Any, vocab: int, max_top_k: Optional[int] = None,
                         use_sparse_topk: bool = True):
    """Per-request ``(top_ks, top_ps, max_top_k bound)`` of SPEC/dflash_utils.py:754-809.

    top-k applies when ``need_top_k_sampling`` (k clamped to [1, V]); on the
    sparse path the k of every row is further clamped to ``max_top_k`` (the
    largest requested k when None, which costs a host read as in the
    reference); top-p applies when ``need_top_p_sampling``.  None = filter off.
    """
    need_top_k = bool(getattr(sampling_info, "need_top_k_sampling", True))
    need_top_p = bool(getattr(sampling_info, "need_top_p_sampling", False))
    ks = None
    mk_bound = None
    if need_top_k:
        ks = sampling_info.top_ks.reshape(-1).to(torch.int64).clamp(min=1, max=vocab)
        if use_sparse_topk:
            mk = int(ks.max().item()) if max_top_k is None else int(max_top_k)
            mk = min(max(mk, 1), vocab)
            if mk < vocab:
                ks = ks.clamp(max=mk)
                mk_bound = mk
    ps = sampling_info.top_ps if need_top_p else None
    return ks, ps, mk_bound

"""ctypes binding of ``liblongspark_amd.so`` (the C ABI in ``include/longspark_amd.h``).

The library is loaded from the package directory; there is no fallback: if it
is missing, importing this module raises with the command that builds it.
Status codes returned by the C ABI are mapped to the exception types the
reference wrappers raise before launching (``ValueError`` for shape, dtype,
alignment, workspace and value errors; ``RuntimeError`` for launch errors).
"""

from __future__ import annotations

import ctypes
from ctypes import c_char_p, c_double, c_float, c_int32, c_int64, c_uint64, c_void_p
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "liblongspark_amd.so"

if not LIB_PATH.exists():
    raise ImportError(
        f"{LIB_PATH} is missing: build the HIP library first with "
        "`python -m longspark_amd.build` (or __graft_entry__.build())")

_lib = ctypes.CDLL(str(LIB_PATH))

LS_OK, LS_ERR_SHAPE, LS_ERR_DTYPE, LS_ERR_ALIGN, LS_ERR_LAUNCH, LS_ERR_WORKSPACE, LS_ERR_VALUE = range(7)
LS_F32, LS_BF16, LS_F16, LS_I32, LS_I64 = range(5)

_DTYPES = {
    torch.float32: LS_F32,
    torch.bfloat16: LS_BF16,
    torch.float16: LS_F16,
    torch.int32: LS_I32,
    torch.int64: LS_I64,
}

P, I32, I64, U64, F32, F64 = c_void_p, c_int32, c_int64, c_uint64, c_float, c_double

class VerifySampleArgs(ctypes.Structure):
    """Mirror of ``ls_verify_sample_args`` (include/longspark_amd.h)."""
    _fields_ = [
        ("logits", P), ("logits_dtype", I32), ("logits_row_stride", I64),
        ("candidates", P), ("candidates_dtype", I32), ("cand_stride_b", I64), ("cand_stride_k", I64),
        ("cand_first_col", I32),
        ("batch", I64), ("width", I32), ("vocab", I64),
        ("temperatures", P), ("top_ks", P), ("top_ps", P), ("min_ps", P), ("max_top_k", I32),
        ("pen_bits", P), ("pen_rank", P), ("pen_words_stride", I64), ("pen_add", P), ("pen_add_stride", I64),
        ("pen_repetition", P), ("pen_verify_quirk", I32), ("pen_nonpositive", P),
        ("vocab_mask", P), ("mask_row_stride", I64), ("mask_per_request", I32),
        ("q_mode", I32), ("draft_token_probs", P), ("dtp_stride_b", I64),
        ("draft", P), ("draft_dtype", I32), ("draft_stride_b", I64), ("draft_stride_k", I64),
        ("draft_temperatures", P), ("draft_top_ks", P), ("draft_top_ps", P), ("draft_min_ps", P),
        ("uniforms", P), ("uniform_stride_b", I64), ("final_uniforms", P),
        ("accept_lens", P), ("bonus", P), ("p_cand_out", P), ("status", P),
        ("timing_events", P), ("scan_hint", I32),
        ("cutoff_verify_lens", P), ("cap_trim", P),
    ]


class TargetProbsArgs(ctypes.Structure):
    """Mirror of ``ls_target_probs_args``."""
    _fields_ = [
        ("logits", P), ("logits_dtype", I32), ("logits_row_stride", I64),
        ("batch", I64), ("rows_per_request", I32), ("vocab", I64),
        ("temperatures", P), ("top_ks", P), ("top_ps", P), ("min_ps", P), ("max_top_k", I32),
        ("out", P), ("out_row_stride", I64), ("status", P), ("scan_hint", I32),
    ]


class ChainSamplingArgs(ctypes.Structure):
    """Mirror of ``ls_chain_sampling_args``."""
    _fields_ = [
        ("target_probs", P), ("tp_stride_b", I64), ("tp_stride_k", I64),
        ("draft_probs", P), ("dp_stride_b", I64), ("dp_stride_k", I64),
        ("candidates", P), ("candidates_dtype", I32), ("cand_stride_b", I64), ("cand_stride_k", I64),
        ("retrive_index", P), ("retrive_index_dtype", I32), ("ri_stride_b", I64), ("ri_stride_k", I64),
        ("uniforms", P), ("uniform_stride_b", I64), ("final_uniforms", P),
        ("batch", I64), ("width", I32), ("vocab", I64),
        ("predicts", P), ("accept_index", P), ("ai_stride_b", I64), ("ai_stride_k", I64),
        ("accept_token_num", P),
    ]


class KvRows(ctypes.Structure):
    """Mirror of ``ls_kv_rows``."""
    _fields_ = [
        ("base", P), ("layers", P), ("stride_layer", I64), ("stride_b", I64), ("stride_w", I64),
        ("stride_loc", I64), ("stride_h", I64), ("located", I32),
    ]


class SummaryArgs(ctypes.Structure):
    """Mirror of ``ls_summary_args``."""
    _fields_ = [
        ("batch", I64), ("layers", I32), ("q_heads", I32), ("kv_heads", I32), ("rows", I32), ("width", I32),
        ("head_dim", I32), ("dtype", I32), ("softmax_scale", F32), ("softcap", F32),
        ("query", P), ("q_stride_l", I64), ("q_stride_b", I64), ("q_stride_h", I64), ("q_stride_s", I64),
        ("keys", KvRows), ("values", KvRows),
        ("scores", P), ("sc_stride_l", I64), ("sc_stride_b", I64), ("sc_stride_h", I64), ("sc_stride_s", I64),
        ("sc_stride_w", I64),
        ("state_output", P), ("so_stride_c", I64), ("so_stride_l", I64), ("so_stride_h", I64), ("so_stride_s", I64),
        ("state_lse", P), ("sl_stride_c", I64), ("sl_stride_l", I64), ("sl_stride_h", I64), ("sl_stride_s", I64),
        ("state_slots", P),
        ("locs", P), ("locs_dtype", I32), ("locs_stride_b", I64), ("locs_stride_w", I64), ("compact_locs", I32),
        ("accept_offsets", P), ("accept_lens", P),
    ]


class PrefillArgs(ctypes.Structure):
    """Mirror of ``ls_prefill_args``."""
    _fields_ = [
        ("batch", I64), ("layers", I32), ("q_heads", I32), ("kv_heads", I32), ("rows", I32), ("head_dim", I32),
        ("dtype", I32), ("softmax_scale", F32), ("softcap", F32),
        ("query", P), ("q_stride_l", I64), ("q_stride_b", I64), ("q_stride_h", I64), ("q_stride_s", I64),
        ("keys", KvRows), ("values", KvRows),
        ("page_table", P), ("pt_dtype", I32), ("pt_stride_b", I64), ("max_len", I64), ("seq_lens", P),
        ("output", P), ("o_stride_l", I64), ("o_stride_b", I64), ("o_stride_h", I64), ("o_stride_s", I64),
        ("lse", P), ("l_stride_l", I64), ("l_stride_b", I64), ("l_stride_h", I64), ("l_stride_s", I64),
        ("round_output", I32), ("chunk", I32),
    ]


class DraftAttentionArgs(ctypes.Structure):
    """Mirror of ``ls_draft_attention_args``."""
    _fields_ = [
        ("batch", I64), ("q_heads", I32), ("kv_heads", I32), ("softmax_scale", F32),
        ("query", P), ("q_stride_b", I64), ("q_stride_h", I64), ("q_stride_r", I64),
        ("global_keys", P), ("gk_stride_b", I64), ("gk_stride_h", I64), ("gk_stride_g", I64),
        ("global_values", P), ("gv_stride_b", I64), ("gv_stride_h", I64), ("gv_stride_g", I64),
        ("state_slots", P),
        ("local_keys", P), ("lk_stride_b", I64), ("lk_stride_h", I64), ("lk_stride_l", I64),
        ("local_values", P), ("lv_stride_b", I64), ("lv_stride_h", I64), ("lv_stride_l", I64),
        ("local_mask", P), ("lm_stride_b", I64), ("lm_stride_r", I64), ("lm_stride_l", I64),
        ("key_cache", P), ("kc_stride_s", I64), ("kc_stride_h", I64),
        ("value_cache", P), ("vc_stride_s", I64), ("vc_stride_h", I64),
        ("page_table", P), ("pt_stride_b", I64), ("raw_lengths", P),
        ("output", P), ("o_stride_b", I64), ("o_stride_h", I64), ("o_stride_r", I64),
        ("raw_output", P), ("ro_stride_t", I64), ("ro_stride_h", I64),
        ("raw_lse", P), ("rl_stride_t", I64), ("rl_stride_h", I64), ("softcap", F32),
    ]


# name -> (restype, argtypes).  Kept in the order of include/longspark_amd.h.
_SIGNATURES = {
    "ls_last_error": (c_char_p, []),
    "ls_version": (c_char_p, []),
    "ls_verify_greedy_workspace": (I32, [I64, I32, I64, P, P]),
    "ls_verify_greedy": (I32, [P, I32, I64, P, I32, I64, I64, I32, I64, I32, I64, P, P, P, P, P,
                               P, U64, P, U64, P]),
    "ls_verify_greedy_noalloc": (I32, [P, I32, I64, P, I32, I64, I64, I32, I64, I32, I64, P, P, P, P, P, P]),
    "ls_penalty_tables": (I32, [P, I64, P, I64, I32, I64, P, P, P, P, I64, P, I64, P, P, P]),
    "ls_adjust_logits": (I32, [P, I32, I64, I64, I64, I32, P, P, I64, P, I64, P, I32, P, I64, I32, I64, P]),
    "ls_add_request_bias": (I32, [P, I32, I64, I64, I64, I32, P, I64, P, I64, I64, P, I64, I32, P]),
    "ls_apply_token_bitmask": (I32, [P, I32, I64, I64, I64, P, I64, I64, I64, P, I32, I64, P]),
    "ls_verify_sample_workspace": (I32, [I64, I32, I64, I32, P, P]),
    "ls_verify_sample": (I32, [ctypes.POINTER(VerifySampleArgs), P, U64, P, U64, P]),
    "ls_softmax_temp": (I32, [P, I32, I64, I64, I64, P, I32, P, I64, P]),
    "ls_target_probs_workspace": (I32, [I64, I32, I64, I32, P, P]),
    "ls_target_probs": (I32, [ctypes.POINTER(TargetProbsArgs), P, U64, P, U64, P]),
    "ls_decide_acceptance": (I32, [P, I32, I64, I64, P, I64, P, I64, P, I64, I64, I64, I32, I64, P, P, I64, P]),
    "ls_finish_sampling": (I32, [P, I64, P, I64, P, I64, P, I64, I64, P, P]),
    "ls_chain_sampling_workspace": (I32, [I64, I64, P, P]),
    "ls_chain_speculative_sampling": (I32, [ctypes.POINTER(ChainSamplingArgs), P, U64, P, U64, P]),
    "ls_finalize_verify_outputs": (I32, [P, I32, I64, I64, P, I32, I64, P, I32, I64, P, I32, I64, I64, I32, P, P, P,
                                         P]),
    "ls_assign_verify_cache_locs": (I32, [P, I32, P, I32, P, I32, P, I32, I64, P, I64, I64, I64, I32, P]),
    "ls_sample_step_workspace": (I32, [I64, I64, P, P]),
    "ls_sample_step": (I32, [P, I32, I64, I64, I64, P, P, I64, P, P, P, P, U64, P, U64, P]),
    "ls_raw_page_table": (I32, [P, I64, I64, P, I32, P, I32, I64, I32, P, I64, P, P]),
    "ls_ring_page_table": (I32, [P, I32, P, I32, I64, I32, P, I64, P, P]),
    "ls_kv_window_gather": (I32, [P, P, I32, I32, I64, I64, I32, I32, P, I64, P, I32, I32, P, I32, I64, I32,
                                  P, I64, I64, I64, I64, I64, P, P]),
    "ls_ring_append": (I32, [P, P, P, P, I32, I64, I64, I64, P, I32, P, P, P, I64, I32, P]),
    "ls_summary_scores": (I32, [ctypes.POINTER(SummaryArgs), P]),
    "ls_summary_merge": (I32, [ctypes.POINTER(SummaryArgs), P]),
    "ls_summary_update": (I32, [ctypes.POINTER(SummaryArgs), P]),
    "ls_global16_prefill_workspace": (I32, [ctypes.POINTER(PrefillArgs), P]),
    "ls_global16_prefill": (I32, [ctypes.POINTER(PrefillArgs), P, I64, P]),
    "ls_draft_attention": (I32, [ctypes.POINTER(DraftAttentionArgs), P]),
    "ls_draft_merge": (I32, [ctypes.POINTER(DraftAttentionArgs), P]),
}

for _name, (_res, _args) in _SIGNATURES.items():
    _fn = getattr(_lib, _name)
    _fn.restype = _res
    _fn.argtypes = _args


def lib():
    return _lib


def exported_symbols():
    return list(_SIGNATURES)


def check(status: int, what: str) -> None:
    """Raise the reference's exception type for a non-zero C ABI status."""
    if status == LS_OK:
        return
    msg = _lib.ls_last_error().decode(errors="replace")
    if status == LS_ERR_LAUNCH:
        raise RuntimeError(f"{what}: {msg}")
    raise ValueError(f"{what}: {msg}")


def call(name: str, *args) -> None:
    check(getattr(_lib, name)(*args), name)


def dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {t.dtype}") from None


def ptr(t):
    """Device address of a tensor (None for a missing optional tensor)."""
    return None if t is None else t.data_ptr()


def stream_of(device: torch.device):
    """Raw hipStream_t of torch's current stream on ``device``."""
    return torch.cuda.current_stream(device).cuda_stream


def capturing() -> bool:
    """True while torch's current stream is recording a HIP graph."""
    return torch.cuda.is_available() and torch.cuda.is_current_stream_capturing()


def require_cuda(*tensors, what: str) -> torch.device:
    """All given (non-None) tensors must live on one GPU; returns that device."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError(f"{what} requires GPU tensors (got a {t.device} tensor)")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"{what}: tensors on different devices ({dev} vs {t.device})")
    if dev is None:
        raise ValueError(f"{what}: no tensors given")
    return dev


def workspace_sizes(fn_name: str, *args):
    """Call a ``*_workspace`` query; returns (counter_bytes, scratch_bytes)."""
    c, s = ctypes.c_uint64(0), ctypes.c_uint64(0)
    call(fn_name, *args, ctypes.byref(c), ctypes.byref(s))
    return c.value, s.value


class _Workspaces:
    """Scratch and counter buffers kept per (device, stream).

    The counter buffer is zero-filled when (re)allocated and every C ABI call
    leaves it zero, so one buffer serves every entry point on a stream.
    Buffers only grow; growing allocates a larger buffer (zero-filled for
    counters) and keeps the old one alive until the process ends, because a
    HIP graph captured earlier may still launch kernels that use it.  Run
    each op once on the capture stream before capturing (torch's usual
    warm-up), so that capture finds its buffers already sized.
    """

    def __init__(self):
        self._bufs = {}
        self._retired = []

    def _get(self, kind: str, nbytes: int, device: torch.device) -> torch.Tensor:
        key = (kind, device.index, stream_of(device))
        buf = self._bufs.get(key)
        if buf is None or buf.numel() < nbytes:
            if buf is not None:
                self._retired.append(buf)
            n = max(int(nbytes), 4096)
            buf = torch.zeros(n, dtype=torch.uint8, device=device) if kind == "counters" else \
                torch.empty(n, dtype=torch.uint8, device=device)
            self._bufs[key] = buf
        return buf

    def get(self, counter_bytes: int, scratch_bytes: int, device: torch.device):
        """(counters, scratch) uint8 tensors of at least the given sizes."""
        return self._get("counters", counter_bytes, device), self._get("scratch", scratch_bytes, device)


workspaces = _Workspaces()

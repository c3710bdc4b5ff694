"""Recent-window (Raw256) refresh on the GPU: page tables, window gather,
selected-row export and ring append.

Drop-ins for
  * ``build_raw256_page_table`` -- SRT/speculative/global16_raw256_draft_fused.py:372-413,
  * ``ring_page_table``         -- src/longspark/engine/draft.py:14-21,
  * ``gather_selected_kv``      -- src/longspark/engine/state_export.py:14-47 (one rank),
and the gathers those tables feed (the window gather, and the ring append of
src/longspark/engine/draft.py:207-212, 255-259).  ``SRT`` =
``vendor/sglang/python/sglang/srt``.
"""

from __future__ import annotations

import weakref
from typing import Optional, Sequence, Union

import torch

from . import _lib

Layers = Union[torch.Tensor, Sequence[torch.Tensor]]

_INDEX = (torch.int32, torch.int64)


class LayerPointers:
    """Device arrays of per-layer base addresses, one per live set of layer tensors.

    KV pools keep one tensor per layer; the kernels take a device array of
    their base addresses.  The array is built once per distinct set of layer
    tensors (a small host-to-device copy) and reused afterwards.

    An array lives exactly as long as the tensors it points into: each entry
    holds weak references to the storage owners of its layers (the tensor a
    view was taken from), and only entries whose owners have all been freed
    are dropped.  A HIP graph that captured a launch therefore never sees its
    pointer array freed while the pool it points into is alive.

    A host-to-device copy cannot be recorded into a graph, so the first use of
    a pool must come before capture: call :meth:`prepare` (or any op on the
    pool) first.  A lookup during capture that finds no array raises.
    """

    def __init__(self, sweep_every: int = 64):
        self._cache = {}
        self._sweep_every = sweep_every
        self._built = 0

    @staticmethod
    def _addresses(layers: Layers):
        if isinstance(layers, torch.Tensor):
            return tuple(layers.data_ptr() + i * layers.stride(0) * layers.element_size()
                         for i in range(layers.shape[0])), (layers,)
        items = list(layers)
        return tuple(t.data_ptr() for t in items), items

    @staticmethod
    def _owner(t: torch.Tensor) -> torch.Tensor:
        while t._base is not None:
            t = t._base
        return t

    def _sweep(self):
        dead = [k for k, (arr, refs) in self._cache.items() if any(r() is None for r in refs)]
        for k in dead:
            del self._cache[k]

    def get(self, layers: Layers, device: torch.device) -> torch.Tensor:
        addrs, items = self._addresses(layers)
        key = (getattr(device, "index", None), addrs)
        hit = self._cache.get(key)
        if hit is not None and all(r() is not None for r in hit[1]):
            return hit[0]
        if self._capturing():
            raise RuntimeError("KV layer pointer array built during graph capture: call "
                               "longspark_amd.kvwindow.layer_pointers.prepare(layers) before capturing")
        self._built += 1
        if self._built % self._sweep_every == 0:
            self._sweep()
        owners = {id(o): o for o in (self._owner(t) for t in items)}
        refs = tuple(weakref.ref(o) for o in owners.values())
        arr = self._make_array(addrs, device)
        self._cache[key] = (arr, refs)
        return arr

    @staticmethod
    def _capturing() -> bool:
        return _lib.capturing()

    @staticmethod
    def _make_array(addrs, device) -> torch.Tensor:
        return torch.tensor([a if a < 1 << 63 else a - (1 << 64) for a in addrs], dtype=torch.int64, device=device)

    def prepare(self, *layer_sets: Layers) -> None:
        """Build the pointer arrays of the given pools now (before a graph capture)."""
        for layers in layer_sets:
            items = list(layers) if not isinstance(layers, torch.Tensor) else [layers]
            self.get(layers, items[0].device)

    def __len__(self):
        return len(self._cache)


layer_pointers = LayerPointers()


def _layer_list(layers: Layers):
    return [layers[i] for i in range(layers.shape[0])] if isinstance(layers, torch.Tensor) else list(layers)


def _check_layers(layers: Layers, what: str, name: str):
    """Per-layer tensors ``[N, H, D]`` (or one ``[L, N, H, D]`` tensor) of one dtype and layout."""
    items = _layer_list(layers)
    if not items:
        raise ValueError(f"{what}: {name} needs at least one layer")
    first = items[0]
    for t in items:
        if t.ndim != 3 or t.shape[1:] != first.shape[1:] or t.dtype != first.dtype or t.stride() != first.stride():
            raise ValueError(f"{what}: {name} layers must share shape [N, H, D], dtype and strides")
        if t.stride(2) != 1:
            raise ValueError(f"{what}: {name} rows must have a contiguous head dimension")
    return items


def build_raw256_page_table(*, req_to_token: torch.Tensor, req_pool_indices: torch.Tensor, seq_lens: torch.Tensor,
                            page_table: torch.Tensor, raw_lengths: torch.Tensor):
    """Fill ``page_table[b, i] = req_to_token[slot_b, seq_b - raw_b + i]`` (0 past
    ``raw_b = min(seq_b, window)``) and ``raw_lengths``; window = ``page_table.shape[1]``
    (256 in the reference contract).  In place; returns ``(page_table, raw_lengths)``."""
    what = "build_raw256_page_table"
    dev = _lib.require_cuda(req_to_token, req_pool_indices, seq_lens, page_table, raw_lengths, what=what)
    batch = int(req_pool_indices.shape[0])
    if (req_to_token.dtype != torch.int32 or req_to_token.ndim != 2
            or req_pool_indices.dtype not in _INDEX or req_pool_indices.shape != (batch,)
            or seq_lens.dtype not in _INDEX or seq_lens.shape != (batch,)
            or page_table.dtype != torch.int32 or page_table.ndim != 2 or page_table.shape[0] != batch
            or page_table.stride(1) != 1
            or raw_lengths.dtype != torch.int32 or raw_lengths.shape != (batch,) or not raw_lengths.is_contiguous()):
        raise ValueError("Raw256 page-table tensors violate the production contract")
    _lib.call("ls_raw_page_table", req_to_token.data_ptr(), req_to_token.stride(0), req_to_token.stride(1),
              req_pool_indices.data_ptr(), _lib.dtype_code(req_pool_indices), seq_lens.data_ptr(),
              _lib.dtype_code(seq_lens), batch, page_table.shape[1], page_table.data_ptr(), page_table.stride(0),
              raw_lengths.data_ptr(), _lib.stream_of(dev))
    return page_table, raw_lengths


def ring_page_table(slots: torch.Tensor, lengths: torch.Tensor, window: int = 256):
    """Chronological ring rows ``slot * window + (len - raw + i) mod window`` and
    ``raw = min(len, window)``, both int32 (src/longspark/engine/draft.py:14-21)."""
    if slots.ndim != 1 or lengths.shape != slots.shape:
        raise ValueError("ring metadata requires one slot and length per request")
    dev = _lib.require_cuda(slots, lengths, what="ring_page_table")
    if slots.dtype not in _INDEX or lengths.dtype not in _INDEX:
        raise ValueError("ring_page_table: slots and lengths must be int32 or int64")
    batch = slots.shape[0]
    slots, lengths = slots.contiguous(), lengths.contiguous()
    pages = torch.empty(batch, window, dtype=torch.int32, device=dev)
    raw = torch.empty(batch, dtype=torch.int32, device=dev)
    _lib.call("ls_ring_page_table", slots.data_ptr(), _lib.dtype_code(slots), lengths.data_ptr(),
              _lib.dtype_code(lengths), batch, window, pages.data_ptr(), pages.stride(0), raw.data_ptr(),
              _lib.stream_of(dev))
    return pages, raw


def gather_window(k_layers: Layers, v_layers: Layers, page_table: torch.Tensor, seq_lens: torch.Tensor, *,
                  page_size: int, window: int = 256, table_rows: Optional[torch.Tensor] = None,
                  out: Optional[torch.Tensor] = None, raw_lengths: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Dense head-major view ``[B, L, 2, H, window, D]`` of each request's last
    ``raw = min(seq, window)`` positions, zero past ``raw``.

    ``k_layers`` / ``v_layers``: per-layer pools ``[N, H, D]`` (a list, or one
    ``[L, N, H, D]`` tensor).  Position t of request b lives at row
    ``page_table[row_b, t // page_size] * page_size + t % page_size`` with
    ``row_b = table_rows[b]`` (default b).  With ``page_size=1`` and
    ``table_rows=req_pool_indices`` the table is SGLang's ``req_to_token``.
    """
    what = "gather_window"
    dev = _lib.require_cuda(page_table, seq_lens, table_rows, out, raw_lengths, what=what)
    ks, vs = _check_layers(k_layers, what, "k_layers"), _check_layers(v_layers, what, "v_layers")
    if len(ks) != len(vs) or ks[0].shape[1:] != vs[0].shape[1:] or ks[0].dtype != vs[0].dtype \
            or ks[0].stride() != vs[0].stride():
        raise ValueError(f"{what}: K and V layers must match")
    for t in ks + vs:
        if t.device != dev:
            raise ValueError(f"{what}: KV pools must share the page table's device")
    if page_table.dtype != torch.int32 or page_table.ndim != 2 or page_table.stride(1) != 1:
        raise ValueError(f"{what}: page_table must be int32 [rows, pages] with unit column stride")
    batch = seq_lens.shape[0]
    if seq_lens.dtype not in _INDEX or seq_lens.ndim != 1:
        raise ValueError(f"{what}: seq_lens must be int32/int64 [B]")
    if table_rows is not None and (table_rows.dtype not in _INDEX or table_rows.shape != (batch,)):
        raise ValueError(f"{what}: table_rows must be int32/int64 [B]")
    n_layers, heads, dim = len(ks), ks[0].shape[1], ks[0].shape[2]
    shape = (batch, n_layers, 2, heads, window, dim)
    if out is None:
        out = torch.empty(shape, dtype=ks[0].dtype, device=dev)
    elif out.shape != shape or out.dtype != ks[0].dtype or out.stride(5) != 1:
        raise ValueError(f"{what}: out must be {tuple(shape)} {ks[0].dtype} with contiguous head rows")
    if raw_lengths is not None and (raw_lengths.dtype != torch.int32 or raw_lengths.shape != (batch,)):
        raise ValueError(f"{what}: raw_lengths must be int32 [B]")
    if batch == 0:
        return out
    kp, vp = layer_pointers.get(k_layers, dev), layer_pointers.get(v_layers, dev)
    seq_lens = seq_lens.contiguous()
    table_rows = table_rows.contiguous() if table_rows is not None else None
    _lib.call("ls_kv_window_gather", kp.data_ptr(), vp.data_ptr(), n_layers, _lib.dtype_code(ks[0]),
              ks[0].stride(0), ks[0].stride(1), heads, dim, page_table.data_ptr(), page_table.stride(0),
              _lib.ptr(table_rows), _lib.dtype_code(table_rows) if table_rows is not None else _lib.LS_I32,
              page_size, seq_lens.data_ptr(), _lib.dtype_code(seq_lens), batch, window, out.data_ptr(),
              out.stride(0), out.stride(1), out.stride(2), out.stride(3), out.stride(4), _lib.ptr(raw_lengths),
              _lib.stream_of(dev))
    return out


def gather_selected_kv(k_layers: Layers, v_layers: Layers, locations: torch.Tensor, *,
                       out: Optional[torch.Tensor] = None):
    """Rows ``locations`` of every layer's K and V: returns ``(keys, values)``,
    each ``[L, n, H, D]`` (views of one ``[2, L, n, H, D]`` buffer).

    One-rank form of src/longspark/engine/state_export.py:14-47 (the target's
    accepted-row export, ``key.index_select(0, locations)`` per layer).
    """
    what = "gather_selected_kv"
    dev = _lib.require_cuda(locations, out, what=what)
    if locations.ndim != 1 or locations.numel() == 0 or locations.dtype not in _INDEX:
        raise ValueError("KV export requires selected layers and nonempty 1D locations")
    ks, vs = _check_layers(k_layers, what, "k_layers"), _check_layers(v_layers, what, "v_layers")
    n_layers, heads, dim = len(ks), ks[0].shape[1], ks[0].shape[2]
    n = locations.shape[0]
    shape = (2, n_layers, n, heads, dim)
    if out is None:
        out = torch.empty(shape, dtype=ks[0].dtype, device=dev)
    elif out.shape != shape or not out.is_contiguous() or out.dtype != ks[0].dtype:
        raise ValueError(f"{what}: out must be a contiguous {shape} tensor")
    if ks[0].stride(1) != dim:
        raise ValueError(f"{what}: a token row must hold its heads contiguously")
    row_bytes = heads * dim * ks[0].element_size()
    locations = locations.contiguous()
    # One request of n rows, appended at ring position 0 of a window of n rows:
    # destination row j of layer l is out[kv, l, j].
    dst_k = [out[0, i] for i in range(n_layers)]
    dst_v = [out[1, i] for i in range(n_layers)]
    zero = torch.zeros(1, dtype=torch.int32, device=dev)
    count = torch.full((1,), n, dtype=torch.int32, device=dev)
    _lib.call("ls_ring_append", layer_pointers.get(k_layers, dev).data_ptr(),
              layer_pointers.get(v_layers, dev).data_ptr(), layer_pointers.get(dst_k, dev).data_ptr(),
              layer_pointers.get(dst_v, dev).data_ptr(), n_layers, row_bytes,
              ks[0].stride(0) * ks[0].element_size(), row_bytes, locations.data_ptr(), _lib.dtype_code(locations),
              zero.data_ptr(), zero.data_ptr(), count.data_ptr(), 1, n, _lib.stream_of(dev))
    return out[0], out[1]


def ring_append(ring_keys: Layers, ring_values: Layers, rows_k: Layers, rows_v: Layers, slots: torch.Tensor,
                previous_lengths: torch.Tensor, counts: torch.Tensor, *, window: int = 256,
                src_locs: Optional[torch.Tensor] = None) -> None:
    """In place: request b's ``counts[b]`` new rows go to ring rows
    ``slots[b] * window + (previous_lengths[b] + j) mod window`` of every layer.

    Source rows are packed request after request (``rows_*`` ``[L, n, H, D]``
    as exported, src/longspark/engine/draft.py:255-259), or, with
    ``src_locs``, read straight from the target pool at those locations (the
    export and the append fused into one copy).
    """
    what = "ring_append"
    dev = _lib.require_cuda(slots, previous_lengths, counts, src_locs, what=what)
    rk, rv = _check_layers(ring_keys, what, "ring_keys"), _check_layers(ring_values, what, "ring_values")
    sk, sv = _check_layers(rows_k, what, "rows_k"), _check_layers(rows_v, what, "rows_v")
    if not (len(rk) == len(rv) == len(sk) == len(sv)):
        raise ValueError(f"{what}: layer counts differ")
    if rk[0].shape[1:] != sk[0].shape[1:] or rk[0].dtype != sk[0].dtype or rk[0].stride() != rv[0].stride() \
            or sk[0].stride() != sv[0].stride():
        raise ValueError(f"{what}: ring and source rows must match in shape, dtype and layout")
    heads, dim = rk[0].shape[1], rk[0].shape[2]
    if rk[0].stride(1) != dim or sk[0].stride(1) != dim:
        raise ValueError(f"{what}: a token row must hold its heads contiguously")
    batch = slots.shape[0]
    for name, t in (("slots", slots), ("previous_lengths", previous_lengths), ("counts", counts)):
        if t.dtype != torch.int32 or t.shape != (batch,):
            raise ValueError(f"{what}: {name} must be int32 [B]")
    if src_locs is not None and (src_locs.ndim != 1 or src_locs.dtype not in _INDEX):
        raise ValueError(f"{what}: src_locs must be a 1-D int32/int64 tensor")
    es = rk[0].element_size()
    _lib.call("ls_ring_append", layer_pointers.get(rows_k, dev).data_ptr(), layer_pointers.get(rows_v, dev).data_ptr(),
              layer_pointers.get(ring_keys, dev).data_ptr(), layer_pointers.get(ring_values, dev).data_ptr(),
              len(rk), heads * dim * es, sk[0].stride(0) * es, rk[0].stride(0) * es, _lib.ptr(src_locs),
              _lib.dtype_code(src_locs) if src_locs is not None else _lib.LS_I32,
              slots.contiguous().data_ptr(), previous_lengths.contiguous().data_ptr(),
              counts.contiguous().data_ptr(), batch, window, _lib.stream_of(dev))

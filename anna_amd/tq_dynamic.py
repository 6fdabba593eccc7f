"""The TurboQuant layers of Qwen3DynamicCache, batched: a drop-in for the reference's
``Qwen3DynamicCache._update_turboquant_layer`` / ``update`` and
``turboquant_single_token_decode_attention`` (src/anna/model/ops.py:618-661, 663-672, 1024-1072).

The reference keeps one ``TurboQuantKVRow`` per (layer, sequence) and loops over them: every
decode step appends row by row and decodes row by row.  Here the rows of one layer live in one
slab of batched tensors ([batch, kv_heads, capacity, ...]), so

  * ``update`` with one new token per sequence (the decode step) quantizes every sequence's
    overflowing window token in one call per quantizer, whatever the batch size;
  * ``turboquant_single_token_decode_attention`` is one split-KV decode over the whole batch with
    per-row lengths on the device (``anna_mi_gqa_decode_splitkv`` with ``seq_lengths``).

Row semantics are the reference row's (turboquant.py:1027-1140): the newest ``residual_len``
tokens stay dense, older tokens are quantized in order; keys use the inner-product quantizer
(mse indices, norms, QJL signs, residual norms) and are decoded from their reconstruction in the
cache dtype (turboquant.py:1098-1111), values use the min/max groups (turboquant.py:199-230).
``key_quantizer="mse"`` keeps TQ-MSE key codes instead and scores them against the rotated query.
The state of a row equals, bit for bit, that of a ``TurboQuantKVRow`` fed the same appends
(every quantizer is per vector), and ``turboquant_rows[layer][b].clone()`` returns such a row.

The window of a sequence is a ring: token j sits in slot j % residual_len.  Attention does not
depend on token order, and while a sequence is shorter than the window its tokens fill slots
0..length-1, which is the layout the decode's ``seq_lengths`` contract reads.
"""

from __future__ import annotations

import torch

from . import _lib
from . import fused_ops
from .turboquant import (
    VALID_KV_CACHE_QUANT_BITS,
    _DECODE_BLOCK_SIZE,
    TurboQuantKeyState,
    TurboQuantKVRow,
    _next_capacity,
    _quantize_turboquant_keys,
    _require_rocm,
    _resolve_value_group_size,
    dequantize_turboquant_keys,
    get_turboquant_quantizer,
    quantize_turboquant_values,
)


class _LayerSlab:
    """Storage of every sequence of one layer.  Per (sequence, KV head): `capacity` quantized
    slots and a window ring of `residual_len` dense tokens; lengths on the host and the device."""

    def __init__(self, *, batch: int, heads: int, head_dim: int, dtype, device, bits: int, residual_len: int,
                 key_quantizer: str, value_group_size: int | None):
        self.batch, self.heads, self.head_dim = batch, heads, head_dim
        self.dtype, self.device, self.bits = dtype, device, bits
        self.R = residual_len
        self.key_quantizer = key_quantizer
        self.value_group_size = value_group_size or _resolve_value_group_size(head_dim)
        self.capacity = 0
        self.lengths = [0] * batch
        self.seq_lengths = torch.zeros((batch,), dtype=torch.int32, device=device)
        B, H, R, D = batch, heads, residual_len, head_dim
        self.rk = torch.zeros((B, H, R, D), dtype=dtype, device=device)
        self.rv = torch.zeros((B, H, R, D), dtype=dtype, device=device)
        self._ws: dict[str, torch.Tensor] = {}

    # ---- lengths
    def qlen(self, b: int) -> int:
        return max(0, self.lengths[b] - self.R)

    def rlen(self, b: int) -> int:
        return min(self.lengths[b], self.R)

    # ---- quantized storage
    def _grow(self, required: int) -> None:
        if required <= self.capacity:
            return
        cap = _next_capacity(self.capacity, required)
        B, H, D, dev = self.batch, self.heads, self.head_dim, self.device
        sb = 2 if self.bits == 2 else 4
        shapes = {
            "vdata": ((B, H, cap, D * sb // 8), torch.uint8),
            "vscales": ((B, H, cap, D // self.value_group_size), self.dtype),
            "vzeros": ((B, H, cap, D // self.value_group_size), self.dtype),
        }
        if self.key_quantizer == "ip":
            shapes.update(kidx=((B, H, cap, D), torch.uint8), knorms=((B, H, cap), torch.float32),
                          kqjl=((B, H, cap, D), torch.uint8), krn=((B, H, cap), torch.float32),
                          kdense=((B, H, cap, D), self.dtype))
        else:
            shapes.update(kcodes=((B, H, cap, D * sb // 8), torch.uint8), knorms=((B, H, cap), torch.float16))
        old = self.capacity
        for name, (shape, dt) in shapes.items():
            t = torch.empty(shape, dtype=dt, device=dev)
            if old > 0:
                t[:, :, :old].copy_(getattr(self, name))
            setattr(self, name, t)
        self.capacity = cap

    def _quantize(self, keys: torch.Tensor, values: torch.Tensor) -> dict[str, torch.Tensor]:
        """keys/values [n, D] -> the per-token fields, each [n, ...]."""
        n, D = keys.shape
        v = quantize_turboquant_values(values.reshape(n, 1, D), bits=self.bits, group_size=self.value_group_size)
        out = {"vdata": v.data.reshape(n, -1), "vscales": v.scales.reshape(n, -1), "vzeros": v.zeros.reshape(n, -1)}
        if self.key_quantizer == "ip":
            st = _quantize_turboquant_keys(keys.reshape(n, 1, D), bits=self.bits, device=self.device)
            out.update(kidx=st.mse_indices.reshape(n, D), knorms=st.norms.reshape(n), kqjl=st.qjl_signs.reshape(n, D),
                       krn=st.residual_norms.reshape(n),
                       kdense=dequantize_turboquant_keys(st, bits=self.bits, device=self.device,
                                                         dtype=self.dtype).reshape(n, D))
        else:
            codes, norms = get_turboquant_quantizer(head_dim=D, bits=self.bits, device=self.device).quantize(keys)
            out.update(kcodes=codes, knorms=norms)
        return out

    def store_range(self, b: int, start: int, keys: torch.Tensor, values: torch.Tensor) -> None:
        """Quantize keys/values [H, t, D] of sequence b into its slots start..start+t-1."""
        H, t, D = keys.shape
        self._grow(start + t)
        fields = self._quantize(keys.reshape(H * t, D), values.reshape(H * t, D))
        for name, f in fields.items():
            getattr(self, name)[b, :, start:start + t].copy_(f.reshape(H, t, *f.shape[1:]))

    def store_scatter(self, rows: torch.Tensor, slots: torch.Tensor, keys: torch.Tensor, values: torch.Tensor) -> None:
        """Quantize one token per listed sequence: keys/values [n, H, D] into slot slots[i] of
        sequence rows[i] (device index tensors)."""
        n, H, D = keys.shape
        fields = self._quantize(keys.reshape(n * H, D), values.reshape(n * H, D))
        for name, f in fields.items():
            getattr(self, name)[rows, :, slots] = f.reshape(n, H, *f.shape[1:])

    # ---- the window ring
    def window(self, b: int) -> tuple[torch.Tensor, torch.Tensor]:
        """The dense window of sequence b in token order, [H, rlen, D] each."""
        L, r = self.lengths[b], self.rlen(b)
        if r == 0:
            empty = self.rk.new_empty((self.heads, 0, self.head_dim))
            return empty, empty
        slots = torch.arange(L - r, L, device=self.device) % self.R
        return self.rk[b][:, slots], self.rv[b][:, slots]

    # ---- appends
    def append(self, keys: torch.Tensor, values: torch.Tensor) -> None:
        """keys/values [B, H, T, D]: T new tokens for every sequence (reference row append,
        turboquant.py:1027-1140, for all rows)."""
        B, H, T, D = keys.shape
        if T == 1 and all(n >= self.R for n in self.lengths):
            # decode step: each sequence's oldest window token (slot L % R) is quantized into
            # slot L - R and the new token takes its place in the ring
            self._grow(max(self.lengths) - self.R + 1)
            rows = torch.arange(B, device=self.device)
            lens = self.seq_lengths.long()
            ring = lens % self.R
            self.store_scatter(rows, lens - self.R, self.rk[rows, :, ring], self.rv[rows, :, ring])
            self.rk[rows, :, ring] = keys[:, :, 0]
            self.rv[rows, :, ring] = values[:, :, 0]
        else:
            for b in range(B):
                self._append_row(b, keys[b], values[b])
        self.lengths = [n + T for n in self.lengths]
        self.seq_lengths += T

    def _append_row(self, b: int, keys: torch.Tensor, values: torch.Tensor) -> None:
        H, T, D = keys.shape
        L, R = self.lengths[b], self.R
        wk, wv = self.window(b)
        seq_k = torch.cat((wk, keys), dim=1)
        seq_v = torch.cat((wv, values), dim=1)
        overflow = seq_k.shape[1] - R
        if overflow > 0:
            self.store_range(b, self.qlen(b), seq_k[:, :overflow], seq_v[:, :overflow])
            seq_k, seq_v = seq_k[:, overflow:], seq_v[:, overflow:]
        n = seq_k.shape[1]
        slots = torch.arange(L + T - n, L + T, device=self.device) % R
        self.rk[b][:, slots] = seq_k
        self.rv[b][:, slots] = seq_v

    # ---- decode
    def _workspace(self, name: str, shape, dtype) -> torch.Tensor:
        numel = torch.Size(shape).numel()
        t = self._ws.get(name)
        if t is None or t.numel() < numel:
            t = torch.empty(max(numel, 2 * (0 if t is None else t.numel())), dtype=dtype, device=self.device)
            self._ws[name] = t
        return t[:numel].view(shape)

    def decode(self, query: torch.Tensor, *, scaling: float, gate: torch.Tensor | None,
               rows: slice = slice(None)) -> torch.Tensor:
        """query [b, Hq, 1, D] for the sequences `rows` -> output of the same shape: one split-KV
        decode over [quantized slots ++ window ring] with the device lengths."""
        b = query.shape[0]
        hq, D = int(query.shape[1]), self.head_dim
        C = self.capacity
        qn = get_turboquant_quantizer(head_dim=D, bits=self.bits, device=self.device)
        if self.key_quantizer == "ip":
            kargs = dict(key=self.kdense[rows] if C else None, key_format=fused_ops.KEYS_DENSE)
        else:
            kargs = dict(key=self.kcodes[rows] if C else None, key_format=fused_ops.KEYS_TQ_MSE,
                         key_norms=self.knorms[rows] if C else None)
        out = torch.empty_like(query)
        args = fused_ops.decode_args(
            query=query, len1=C, **kargs, key_bits=self.bits,
            value=self.vdata[rows] if C else None, value_format=fused_ops.VALUES_MINMAX,
            value_scales=self.vscales[rows] if C else None, value_zeros=self.vzeros[rows] if C else None,
            value_bits=self.bits, value_group_size=self.value_group_size,
            rotation=qn.rotation, rotation_t=qn.rotation_t, key_centroids=qn.centroids, rotation_signs=qn.signs,
            query_rot=self._workspace("qrot", (b, hq, D), torch.float32),
            residual_key=self.rk[rows], residual_value=self.rv[rows], scaling=scaling,
            block_size=_DECODE_BLOCK_SIZE, gate=gate, output=out,
            partial_stats=self._workspace("ps", (b, hq, 1, 2), torch.float32),
            partial_values=self._workspace("pv", (b, hq, 1, D), torch.float32),
            seq_lengths=self.seq_lengths[rows])
        nblk = fused_ops.decode_num_blocks(args)
        args.partial_stats = _lib.view(self._workspace("ps", (b, hq, nblk, 2), torch.float32))
        args.partial_values = _lib.view(self._workspace("pv", (b, hq, nblk, D), torch.float32))
        args.partial_capacity = nblk
        fused_ops.run_decode(args, query)
        lens = self.lengths[rows]
        if 0 in lens:  # the reference returns zeros for an empty row
            for i, n in enumerate(lens):
                if n == 0:
                    out[i].zero_()
        return out


class TurboQuantSlabRow:
    """One sequence of a layer slab, with the reference row's read API (length properties,
    materialize, decode_attention, clone)."""

    def __init__(self, slab: _LayerSlab, b: int):
        self._slab, self._b = slab, b

    @property
    def bits(self) -> int:
        return self._slab.bits

    @property
    def residual_len(self) -> int:
        return self._slab.R

    @property
    def initialized(self) -> bool:
        return True

    @property
    def length(self) -> int:
        return self._slab.lengths[self._b]

    @property
    def quantized_length(self) -> int:
        return self._slab.qlen(self._b)

    @property
    def residual_length(self) -> int:
        return self._slab.rlen(self._b)

    def key_state(self) -> TurboQuantKeyState:
        """The inner-product key state of the quantized prefix (reference TurboQuantKeyState)."""
        s, b, n = self._slab, self._b, self.quantized_length
        if s.key_quantizer != "ip":
            raise RuntimeError("key_state() needs key_quantizer='ip'")
        if n == 0:
            raise RuntimeError("the row has no quantized tokens")
        return TurboQuantKeyState(mse_indices=s.kidx[b, :, :n], norms=s.knorms[b, :, :n, None],
                                  qjl_signs=s.kqjl[b, :, :n], residual_norms=s.krn[b, :, :n, None])

    def materialize(self, *, device=None, dtype=None):
        s, b, n = self._slab, self._b, self.quantized_length
        H, D = s.heads, s.head_dim
        kp, vp = [], []
        if n > 0:
            if s.key_quantizer == "ip":
                kp.append(s.kdense[b, :, :n])
            else:
                qn = get_turboquant_quantizer(head_dim=D, bits=s.bits, device=s.device)
                kp.append(qn.dequantize(s.kcodes[b, :, :n].reshape(H * n, -1), s.knorms[b, :, :n].reshape(-1),
                                        dtype=s.dtype).view(H, n, D))
            vp.append(fused_ops.tq_values_dequant(s.vdata[b, :, :n], s.vscales[b, :, :n], s.vzeros[b, :, :n],
                                                  s.bits, s.value_group_size, s.dtype))
        wk, wv = s.window(b)
        keys = torch.cat(kp + [wk], dim=1)
        values = torch.cat(vp + [wv], dim=1)
        if device is not None or dtype is not None:
            keys, values = keys.to(device=device, dtype=dtype), values.to(device=device, dtype=dtype)
        return keys, values

    def decode_attention(self, query: torch.Tensor, *, scaling: float, num_key_value_groups: int,
                         gate: torch.Tensor | None = None) -> torch.Tensor:
        s = self._slab
        _check_query(query[None], gate if gate is None else gate[None], s, num_key_value_groups)
        out = s.decode(query[None], scaling=scaling, gate=None if gate is None else gate[None],
                       rows=slice(self._b, self._b + 1))
        return out[0]

    def clone(self) -> TurboQuantKVRow:
        """An independent TurboQuantKVRow holding this row's state."""
        s, b, n = self._slab, self._b, self.quantized_length
        row = TurboQuantKVRow(bits=s.bits, residual_len=s.R, value_group_size=s.value_group_size,
                              key_quantizer=s.key_quantizer)
        row.device, row.dtype, row.head_dim, row.num_heads = s.device, s.dtype, s.head_dim, s.heads
        if n > 0:
            row._grow(n)
        row._length, row._qlen = self.length, n
        if n > 0:
            pairs = [("_vdata", "vdata"), ("_vscales", "vscales"), ("_vzeros", "vzeros"), ("_knorms", "knorms")]
            if s.key_quantizer == "ip":
                pairs += [("_kcodes", "kidx"), ("_kqjl", "kqjl"), ("_krn", "krn"), ("_kdense", "kdense")]
            else:
                pairs += [("_kcodes", "kcodes")]
            for mine, theirs in pairs:
                getattr(row, mine)[:, :n].copy_(getattr(s, theirs)[b, :, :n])
        wk, wv = s.window(b)
        row._residual_keys, row._residual_values = wk.contiguous(), wv.contiguous()
        return row


def _check_query(query: torch.Tensor, gate, slab: _LayerSlab, groups: int) -> None:
    if query.ndim != 4 or query.shape[2] != 1:
        raise ValueError("TurboQuant decode attention expects query_states shaped [batch, query_heads, 1, head_dim].")
    if gate is not None and gate.shape != query.shape:
        raise ValueError(f"TurboQuant decode gate expects query layout {tuple(query.shape)}, got {tuple(gate.shape)}.")
    if int(query.shape[-1]) != slab.head_dim:
        raise ValueError(f"TurboQuant decode head_dim mismatch: expected {slab.head_dim}, got {int(query.shape[-1])}")
    if int(query.shape[1]) != slab.heads * int(groups):
        raise ValueError(f"Expected {slab.heads * groups} query heads, got {int(query.shape[1])}.")


class TurboQuantDynamicCache:
    """The TurboQuant part of Qwen3DynamicCache (ops.py:342-396): same constructor arguments
    for the KV quantization, same ``layer_lengths`` / ``turboquant_rows`` fields, and the
    ``update`` / ``turboquant_single_token_decode_attention`` / ``get_seq_lengths`` calls.

    ``turboquant_layers``: the layer indices that use TurboQuant storage (the reference takes
    the model's full-attention layers when ``kv_cache_quantization == "turboquant"``); default
    every layer."""

    def __init__(self, num_layers: int, *, batch_size: int = 0, kv_cache_quantization: str = "turboquant",
                 kv_cache_quant_bits: int = 4, kv_cache_residual_len: int = 128, turboquant_layers=None,
                 key_quantizer: str = "ip", value_group_size: int | None = None):
        self.kv_cache_quantization = kv_cache_quantization.strip().lower()
        if self.kv_cache_quantization not in {"none", "turboquant"}:
            raise ValueError(f"Unsupported Qwen3 KV-cache quantization mode: {kv_cache_quantization}")
        self.kv_cache_quant_bits = int(kv_cache_quant_bits)
        if self.kv_cache_quant_bits not in VALID_KV_CACHE_QUANT_BITS:
            raise ValueError(f"Unsupported Qwen3 TurboQuant bit-width: {kv_cache_quant_bits}. "
                             f"Expected one of {sorted(VALID_KV_CACHE_QUANT_BITS)}.")
        if key_quantizer not in ("ip", "mse"):
            raise ValueError(f"key_quantizer must be 'ip' or 'mse', got {key_quantizer!r}")
        self.kv_cache_residual_len = max(1, int(kv_cache_residual_len))
        self.key_quantizer = key_quantizer
        self.value_group_size = value_group_size
        self.num_layers = int(num_layers)
        layers = range(self.num_layers) if turboquant_layers is None else turboquant_layers
        self._turboquant_layer_index_set = (set(int(i) for i in layers)
                                            if self.kv_cache_quantization == "turboquant" else set())
        self.layer_lengths: list[list[int]] = [[0] * batch_size for _ in range(self.num_layers)]
        self.turboquant_rows: list[list[TurboQuantSlabRow | None]] = [[None] * batch_size
                                                                      for _ in range(self.num_layers)]
        self._slabs: list[_LayerSlab | None] = [None] * self.num_layers
        self.seen_tokens = 0

    def uses_turboquant_for_layer(self, layer_idx: int) -> bool:
        return layer_idx in self._turboquant_layer_index_set

    def _ensure_batch_size(self, batch_size: int) -> None:
        if not self.layer_lengths or not self.layer_lengths[0]:
            self.layer_lengths = [[0] * batch_size for _ in range(self.num_layers)]
            self.turboquant_rows = [[None] * batch_size for _ in range(self.num_layers)]
            return
        if len(self.layer_lengths[0]) != batch_size:
            raise ValueError(f"Cache batch size mismatch: expected {len(self.layer_lengths[0])}, got {batch_size}")

    def get_batch_size(self) -> int:
        return len(self.layer_lengths[0]) if self.layer_lengths else 0

    def get_seq_lengths(self, *, device=None) -> torch.Tensor:
        lengths = []
        for b in range(self.get_batch_size()):
            lengths.append(next((self.layer_lengths[i][b] for i in range(self.num_layers)
                                 if self.layer_lengths[i][b] > 0), 0))
        return torch.tensor(lengths, dtype=torch.long, device=device)

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, layer_idx: int, *,
               require_dense_cache: bool = True):
        """key/value_states [batch, kv_heads, T, head_dim] -> (padded keys | None, padded values
        | None, past_lengths), as _update_turboquant_layer (ops.py:618-661)."""
        if not self.uses_turboquant_for_layer(layer_idx):
            raise ValueError(f"Layer {layer_idx} does not use TurboQuant-backed KV storage.")
        if key_states.ndim != 4 or key_states.shape != value_states.shape:
            raise ValueError("TurboQuant update expects key/value states shaped [batch, kv_heads, tokens, head_dim].")
        B, H, T, D = key_states.shape
        self._ensure_batch_size(B)
        _require_rocm(key_states, "TurboQuantDynamicCache")
        past_lengths = torch.tensor(self.layer_lengths[layer_idx], device=key_states.device, dtype=torch.long)
        slab = self._slabs[layer_idx]
        if slab is None:
            slab = _LayerSlab(batch=B, heads=H, head_dim=D, dtype=key_states.dtype, device=key_states.device,
                              bits=self.kv_cache_quant_bits, residual_len=self.kv_cache_residual_len,
                              key_quantizer=self.key_quantizer, value_group_size=self.value_group_size)
            self._slabs[layer_idx] = slab
            self.turboquant_rows[layer_idx] = [TurboQuantSlabRow(slab, b) for b in range(B)]
        elif H != slab.heads or D != slab.head_dim:
            raise ValueError(f"TurboQuantKVRow shape mismatch: expected heads={slab.heads} head_dim={slab.head_dim}, "
                             f"got {tuple(key_states.shape[1:])}")
        if T > 0:
            slab.append(key_states.to(dtype=slab.dtype).detach(), value_states.to(dtype=slab.dtype).detach())
        self.layer_lengths[layer_idx] = list(slab.lengths)
        self.seen_tokens = max(self.get_seq_lengths().tolist(), default=0)
        if not require_dense_cache:
            return None, None, past_lengths
        rows = [r.materialize(device=key_states.device, dtype=key_states.dtype)
                for r in self.turboquant_rows[layer_idx]]
        return _pad_rows([k for k, _ in rows]), _pad_rows([v for _, v in rows]), past_lengths

    def append_row(self, layer_idx: int, batch_idx: int, key_states: torch.Tensor,
                   value_states: torch.Tensor) -> None:
        """Append [kv_heads, T, head_dim] to one sequence of an existing layer (a sequence that
        joins or prefills apart from the others, as TurboQuantKVRow.append does for one row);
        sequence lengths may then differ, which the decode's per-row lengths handle."""
        slab = self._slabs[layer_idx]
        if slab is None:
            raise RuntimeError(f"layer {layer_idx} has no TurboQuant storage yet: call update() first")
        if key_states.ndim != 3 or key_states.shape != value_states.shape or key_states.shape[0] != slab.heads \
                or key_states.shape[2] != slab.head_dim:
            raise ValueError(f"append_row expects [{slab.heads}, tokens, {slab.head_dim}] keys/values")
        T = int(key_states.shape[1])
        if T == 0:
            return
        slab._append_row(batch_idx, key_states.to(dtype=slab.dtype).detach(), value_states.to(dtype=slab.dtype).detach())
        slab.lengths[batch_idx] += T
        slab.seq_lengths[batch_idx] += T
        self.layer_lengths[layer_idx] = list(slab.lengths)

    def turboquant_single_token_decode_attention(self, layer_idx: int, query_states: torch.Tensor, *,
                                                 scaling: float, num_key_value_groups: int,
                                                 gate: torch.Tensor | None = None) -> torch.Tensor:
        """[batch, query_heads, 1, head_dim] -> the same shape: every sequence in one decode
        call (the reference loops TurboQuantKVRow.decode_attention over the rows)."""
        if not self.uses_turboquant_for_layer(layer_idx):
            raise ValueError(f"Layer {layer_idx} does not use TurboQuant-backed KV storage.")
        if query_states.ndim != 4 or query_states.shape[2] != 1:
            raise ValueError("TurboQuant decode attention expects query_states shaped [batch, query_heads, 1, head_dim].")
        if gate is not None and gate.shape != query_states.shape:
            raise ValueError(f"TurboQuant decode gate expects query layout {tuple(query_states.shape)}, "
                             f"got {tuple(gate.shape)}.")
        slab = self._slabs[layer_idx]
        if slab is None:
            return query_states.new_zeros(query_states.shape)
        if int(query_states.shape[0]) != slab.batch:
            raise ValueError(f"Cache batch size mismatch: expected {slab.batch}, got {int(query_states.shape[0])}")
        _check_query(query_states, gate, slab, num_key_value_groups)
        return slab.decode(query_states, scaling=scaling, gate=gate)


def _pad_rows(rows: list[torch.Tensor]) -> torch.Tensor:
    """Rows [H, L_b, D] -> zero-padded [B, H, max L_b, D] (reference _pad_cache_rows, ops.py:443-454)."""
    m = max(int(r.shape[1]) for r in rows)
    out = rows[0].new_zeros((len(rows), rows[0].shape[0], m, rows[0].shape[2]))
    for b, r in enumerate(rows):
        out[b, :, : r.shape[1]].copy_(r)
    return out

"""Page-size-1 MLA latent cache in the reference's ``kv_data`` layout.

The reference builds its caches whole from one bf16 buffer
(competitor_submissions/mi355x_reference/reference.py:311-321, layout in
competitor_submissions/mi355x_reference/README.md:57-81) and addresses them
with ``kv_indices = arange`` (reference.py:245).  A serving loop instead
appends a few tokens per sequence per step; ``KVCache`` does that on the
device with ``mla_append_kv`` and hands out the same tuple the decode takes:

* ``kv_data()``  -> ``{"fp8": (e4m3fn [cap,1,576], scale [1] f32),
  "mxfp4": (fp4x2 [cap,1,288], e8m0 [cap, scale_cols])}``
* ``indices(seq_ids)`` -> ``(kv_indptr, kv_indices)`` int32 on the device.

Cache rows (slots) come from a host free list; a sequence's slots need not be
contiguous, which is what ``kv_indices`` expresses.  The fp8 scale is
per-tensor: given at construction, or taken from the first append (the
prefill) by the whole-buffer rule ``bf16(max|x| / 448)``.  Later tokens are
quantized with that scale; a token whose magnitude exceeds ``448 * scale``
saturates, which ``fp8_saturated()`` reports from the device-side running
``max|x|``.  The mxfp4 cache has per-32-element scales and never saturates.

Appending is stream-ordered on torch's current stream; the slot bookkeeping is
host-only (the allocator and the per-sequence lists), so ``indices`` copies one
int32 list to the device per call.
"""
from __future__ import annotations

import struct

import torch

from . import ops

QK_DIM = 576
FP4_ROW = 288
MX_BLOCKS = 18
FP8_MAX = 448.0


def _bf16_bits_to_float(bits: int) -> float:
    return struct.unpack("<f", struct.pack("<I", (bits & 0xFFFF) << 16))[0]


class KVCache:
    """Device-resident fp8 and/or mxfp4 latent cache with a slot allocator."""

    def __init__(self, capacity: int, formats=("fp8", "mxfp4"), device="cuda", scale_cols: int = MX_BLOCKS,
                 fp8_scale: float | None = None):
        if capacity < 1:
            raise ValueError("capacity must be >= 1")
        formats = tuple(formats)
        if not formats or any(f not in ("fp8", "mxfp4") for f in formats):
            raise ValueError("formats must be a non-empty subset of ('fp8', 'mxfp4')")
        if scale_cols < MX_BLOCKS:
            raise ValueError(f"scale_cols must be >= {MX_BLOCKS}")
        self.capacity = int(capacity)
        self.device = torch.device(device)
        self.formats = formats
        self.fp8 = self.fp8_scale = self.fp4 = self.fp4_scales = None
        if "fp8" in formats:
            self.fp8 = torch.zeros((capacity, 1, QK_DIM), dtype=torch.float8_e4m3fn, device=self.device)
            self.fp8_scale = torch.zeros(1, dtype=torch.float32, device=self.device)
            if fp8_scale is not None:
                if not fp8_scale > 0:
                    raise ValueError("fp8_scale must be positive")
                self.fp8_scale.fill_(float(fp8_scale))
        if "mxfp4" in formats:
            self.fp4 = torch.zeros((capacity, 1, FP4_ROW), dtype=torch.uint8, device=self.device)
            self.fp4_scales = torch.full((capacity, scale_cols), 127, dtype=torch.uint8, device=self.device)
        self._scale_set = fp8_scale is not None or self.fp8 is None
        self.amax_bits = torch.zeros(1, dtype=torch.int32, device=self.device)
        self._free = list(range(self.capacity - 1, -1, -1))  # pop() hands out low slots first
        self._seqs: dict = {}

    # ---- slot allocation -----------------------------------------------------
    @property
    def free_slots(self) -> int:
        return len(self._free)

    def seq_len(self, seq_id) -> int:
        return len(self._seqs.get(seq_id, ()))

    def allocate(self, n: int) -> list:
        if n > len(self._free):
            raise MemoryError(f"KV cache full: {n} slots asked, {len(self._free)} free of {self.capacity}")
        return [self._free.pop() for _ in range(n)]

    def release(self, seq_id) -> None:
        """Return a sequence's slots to the free list (their bytes are left as they are)."""
        slots = self._seqs.pop(seq_id, [])
        self._free.extend(reversed(slots))

    # ---- writing -------------------------------------------------------------
    def calibrate_fp8(self, x: torch.Tensor) -> None:
        """Set the fp8 scale from ``x`` by the whole-buffer rule (reference.py:76-78)."""
        if self.fp8 is None:
            raise ValueError("this cache has no fp8 part")
        _, scale = ops.quant_fp8_per_tensor(x.reshape(-1, QK_DIM))
        self.fp8_scale.copy_(scale)
        self._scale_set = True

    def write(self, x: torch.Tensor, slots: torch.Tensor | None) -> None:
        """Write tokens into given device slots (int32 [n]; negative = skip)."""
        if not self._scale_set:
            self.calibrate_fp8(x)
        ops.append_kv(x, slots,
                      fp8=None if self.fp8 is None else (self.fp8, self.fp8_scale),
                      mxfp4=None if self.fp4 is None else (self.fp4, self.fp4_scales),
                      amax=self.amax_bits)

    def append(self, seq_id, x: torch.Tensor) -> torch.Tensor:
        """Append tokens ``x`` ([n, 576] or [n, 1, 576] bf16) to sequence ``seq_id``.

        Returns the device int32 slots they went to.
        """
        n = x.numel() // QK_DIM
        if x.shape[-1] != QK_DIM or n * QK_DIM != x.numel():
            raise ValueError("x must be [n, 576] or [n, 1, 576]")
        slots = self.allocate(n)
        slots_d = torch.tensor(slots, dtype=torch.int32).to(self.device)
        try:
            self.write(x, slots_d)
        except Exception:
            self._free.extend(reversed(slots))
            raise
        self._seqs.setdefault(seq_id, []).extend(slots)
        return slots_d

    # ---- reading -------------------------------------------------------------
    def indices(self, seq_ids):
        """(kv_indptr [S+1], kv_indices [sum L]) int32 on the device for these sequences."""
        lens, flat = [0], []
        for s in seq_ids:
            sl = self._seqs.get(s, [])
            flat.extend(sl)
            lens.append(lens[-1] + len(sl))
        kv_indptr = torch.tensor(lens, dtype=torch.int32).to(self.device)
        kv_indices = torch.tensor(flat if flat else [0], dtype=torch.int32).to(self.device)
        return kv_indptr, kv_indices

    def kv_data(self) -> dict:
        """The caches in the reference's ``kv_data`` layout (views, no copies)."""
        d = {}
        if self.fp8 is not None:
            d["fp8"] = (self.fp8, self.fp8_scale)
        if self.fp4 is not None:
            d["mxfp4"] = (self.fp4.view(torch.float4_e2m1fn_x2), self.fp4_scales.view(torch.float8_e8m0fnu))
        return d

    def fp8_saturated(self) -> bool:
        """True if a written token was clamped: bf16(max|x| / scale) > 448 (synchronizes the host)."""
        if self.fp8 is None:
            return False
        amax = torch.tensor([_bf16_bits_to_float(int(self.amax_bits.item()))], dtype=torch.float32)
        y = (amax / self.fp8_scale.cpu()).to(torch.bfloat16)
        return bool(y.float().item() > FP8_MAX)

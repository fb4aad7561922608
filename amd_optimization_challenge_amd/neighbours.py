"""The steps on either side of the absorbed decode (DeepSeek-style MLA).

Upstream, W_UK absorption turns a head's no-rope query into the latent space
the cache lives in: q_latent[b, h] = q_nope[b, h] @ W_UK[h] (128 -> 512), and
the decode's Q row is [q_latent, q_rope] (512 + 64 = 576).  Downstream, the
decode's latent output is lifted back by v_up_proj: y[b, h] = o[b, h] @ W_UV[h]
(512 -> 128), optionally quantized to per-tensor FP8 for the next GEMM (the
fusion vLLM does for this layer, mixed-mla/README.md:213-217).  The shared
MXFP4 quantizer of the mxfp4-mm / mxfp4-moe tasks is ``ops.pack_mxfp4`` (any
[rows, cols] bf16 with cols % 32 == 0).

Both products are per-head batched GEMMs with M = batch (tens to hundreds of
rows), dominated by streaming the weights once; they run as plain library
GEMMs (``torch.bmm``, hipBLASLt on ROCm, f32 accumulation) with contiguous
operands.  The FP8 step is this package's bit-exact per-tensor quantizer.
"""
from __future__ import annotations

import torch

from . import ops

QK_NOPE = 128   # DeepSeek-V3/R1 qk_nope_head_dim
QK_ROPE = 64    # qk_rope_head_dim
LATENT = 512    # kv_lora_rank
V_HEAD = 128    # v_head_dim


def _check(*args) -> None:
    """args: (tensor, name, shape) triples; dtypes and shapes first, then devices."""
    for x, name, shape in args:
        if x.dtype != torch.bfloat16:
            raise ValueError(f"{name} must be bfloat16")
        if x.dim() != len(shape) or any(d != s for d, s in zip(x.shape, shape)):
            raise ValueError(f"{name} must have shape {tuple(shape)}, got {tuple(x.shape)}")
    for x, name, _ in args:
        if x.device.type != "cuda":
            raise ValueError(f"{name} must be a CUDA (HIP) tensor")


def absorb_q(q_nope: torch.Tensor, q_rope: torch.Tensor, w_uk: torch.Tensor) -> torch.Tensor:
    """q_nope [B, H, 128], q_rope [B, H, 64], w_uk [H, 128, 512] (bf16) -> the
    decode's Q [B, H, 576] bf16 = [q_nope[b, h] @ w_uk[h], q_rope[b, h]]."""
    B, H = q_nope.shape[0], q_nope.shape[1]
    _check((q_nope, "q_nope", (B, H, QK_NOPE)), (q_rope, "q_rope", (B, H, QK_ROPE)),
           (w_uk, "w_uk", (H, QK_NOPE, LATENT)))
    out = torch.empty((B, H, LATENT + QK_ROPE), dtype=torch.bfloat16, device=q_nope.device)
    lat = torch.bmm(q_nope.transpose(0, 1).contiguous(), w_uk.contiguous())  # [H, B, 512]
    out[..., :LATENT] = lat.transpose(0, 1)
    out[..., LATENT:] = q_rope
    return out


def v_up_proj(o: torch.Tensor, w_uv: torch.Tensor, quant_fp8: bool = False):
    """o [B, H, 512] (the decode output), w_uv [H, 512, 128] (bf16) ->
    y [B, H, 128] bf16 = o[b, h] @ w_uv[h]; with ``quant_fp8`` the pair
    (float8_e4m3fn [B, H, 128], f32 scale [1]) from the per-tensor quantizer."""
    B, H = o.shape[0], o.shape[1]
    _check((o, "o", (B, H, LATENT)), (w_uv, "w_uv", (H, LATENT, V_HEAD)))
    y = torch.bmm(o.transpose(0, 1).contiguous(), w_uv.contiguous()).transpose(0, 1).contiguous()
    if not quant_fp8:
        return y
    return ops.quant_fp8_per_tensor(y)

"""Input/output types of the mixed-mla task (competitor_submissions/mi355x_reference/task.py:4-36).

input_t  = (q [total_q, H, 576] bf16, kv_data dict, qo_indptr [B+1] i32,
            kv_indptr [B+1] i32, config dict)
output_t = [total_q, H, 512] bf16
"""
from typing import TypedDict, TypeVar

import torch

input_t = TypeVar("input_t", bound=tuple[torch.Tensor, dict, torch.Tensor, torch.Tensor, dict])
output_t = TypeVar("output_t", bound=torch.Tensor)


class TestSpec(TypedDict):
    batchsize: int
    qseqlen: int
    kvseqlen: int
    seed: int

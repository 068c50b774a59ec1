"""Helpers for the GPU parity tests."""
import sys

import torch

DEV = torch.device("cuda:0")


def case(msg: str) -> None:
    """Names the case about to run on the GPU, flushed before the launch."""
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def bits16(t: torch.Tensor) -> torch.Tensor:
    return t.detach().cpu().contiguous().view(torch.int16)

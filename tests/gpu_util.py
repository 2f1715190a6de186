"""numpy bit arrays <-> torch device tensors for the GPU tests."""
import numpy as np
import torch


def t16(bits: np.ndarray, dtype: torch.dtype, dev) -> torch.Tensor:
    """uint16 bit patterns -> bf16/f16 device tensor (bit-exact)."""
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(dtype).to(dev)


def t8(bits: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits, dtype=np.uint8)).to(dev)


def ti(a: np.ndarray, dtype, dev) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(dtype).to(dev)


def bits16(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def ptr(t) -> int:
    return 0 if t is None else int(t.data_ptr())


def log_case(msg: str) -> None:
    """Name the case before a GPU step (a fault can end the process)."""
    print(f"[case] {msg}", flush=True)

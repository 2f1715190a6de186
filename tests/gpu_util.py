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


class RawStream:
    """A HIP stream the library has never seen (torch.cuda.Stream() draws from a
    reused pool): created with hipStreamCreate (default priority), wrapped as a
    torch ExternalStream, destroyed on exit after a device synchronisation."""

    def __enter__(self):
        import ctypes
        self._hip = ctypes.CDLL("libamdhip64.so")
        h = ctypes.c_void_p()
        rc = self._hip.hipStreamCreate(ctypes.byref(h))
        assert rc == 0, f"hipStreamCreate: {rc}"
        self.handle = h
        self.stream = torch.cuda.ExternalStream(h.value)
        return self.stream

    def __exit__(self, *exc):
        torch.cuda.synchronize()
        self._hip.hipStreamDestroy(self.handle)
        return False

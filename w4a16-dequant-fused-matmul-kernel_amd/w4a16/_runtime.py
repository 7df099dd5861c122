"""Device plumbing for the HIP kernels: streams, workspaces, device staging.

PyTorch-ROCm supplies device memory and the current stream; every computation
runs in ``libw4a16.so``.  There is no CPU path: without a HIP device these
helpers raise ``RuntimeError``.
"""
from __future__ import annotations

import threading
from contextlib import contextmanager

import torch

from . import _lib

_WS_LOCK = threading.Lock()
_WORKSPACES: dict[tuple[int, int], torch.Tensor] = {}


def require_device() -> torch.device:
    """The current HIP device; RuntimeError if there is none."""
    if not torch.cuda.is_available():
        raise RuntimeError(
            "w4a16 runs on a HIP GPU (MI355X / gfx950) and no HIP device is visible; "
            "there is no CPU fallback")
    return torch.device("cuda", torch.cuda.current_device())


def stream_ptr(device: torch.device) -> int:
    """hipStream_t of torch's current stream on `device`, as an integer."""
    return torch.cuda.current_stream(device).cuda_stream


@contextmanager
def on_device(device: torch.device):
    """Make `device` current for the duration (HIP launches use the current device)."""
    if device.type != "cuda":
        raise RuntimeError(f"expected a HIP device, got {device}")
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if idx == torch.cuda.current_device():
        yield
    else:
        with torch.cuda.device(idx):
            yield


def workspace(device: torch.device, nbytes: int) -> torch.Tensor | None:
    """A workspace of at least `nbytes` for the current stream.

    It holds split-K fp32 partial sums (forced GEMV splits, prefill splits),
    which every call writes before it reads them within the same call, so its
    contents never matter between calls.

    * Eager calls share one buffer per (device, stream): calls on one stream
      are ordered, and a buffer replaced by a larger one goes back to torch's
      stream-ordered caching allocator, which hands it out again only after
      the work already queued on that stream.
    * A call made while the stream is being captured into a HIP graph gets a
      buffer of its own, allocated inside the capture: it comes from the
      graph's private memory pool, so the graph owns it for as long as the
      graph exists, no other graph or eager call can be given it, and
      replaying graphs on different streams at the same time cannot race on
      it.  A later allocation in the same capture may reuse it; replays run
      such work after this call's kernels, as in eager order.  The shared
      eager buffer is never recorded into a graph, so growing or freeing it
      cannot leave a graph pointing at freed memory.
    """
    if nbytes <= 0:
        return None
    if torch.cuda.is_current_stream_capturing():
        return torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)
    key = (device.index if device.index is not None else torch.cuda.current_device(),
           stream_ptr(device))
    with _WS_LOCK:
        ws = _WORKSPACES.get(key)
        if ws is None or ws.numel() < nbytes:
            size = max(nbytes, 1 << 20)
            ws = torch.empty(size, dtype=torch.uint8, device=device)
            _WORKSPACES[key] = ws
        return ws


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stage_to_device(*tensors: torch.Tensor) -> tuple[torch.device, torch.device, list]:
    """Move CPU inputs to the current HIP device.

    Returns (home device, compute device, moved tensors).  Results are copied back
    to the home device by the caller, so API functions that the reference runs
    on any device keep their device semantics while computing on the GPU.
    """
    home = tensors[0].device
    if home.type == "cuda":
        return home, home, list(tensors)
    dev = require_device()
    return home, dev, [t.to(dev) for t in tensors]


def lib():
    return _lib.load()

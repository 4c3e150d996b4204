"""ctypes binding of libactkv_hip.so, the gfx950 C-ABI library (include/actkv.h).

torch is imported first on purpose: torch ships libamdhip64.so.7 and the library's
dependency on that SONAME then resolves to torch's copy, so the process holds one HIP
runtime and device pointers from torch tensors are valid in the library's kernels.

There is no CPU path.  Every wrapper requires ROCm GPU tensors and raises when the
library is missing or a tensor lives on the CPU.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np
import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libactkv_hip.so")

F32, F16, BF16 = 0, 1, 2
REDUCE_MEAN, REDUCE_MAX = 0, 1
WS_KEEP_MASK = 0
ERR_WORKSPACE = 3
KEEP_MASK_SCRATCH_BYTES = 8 << 20       # the static device scratch of actkv_keep_mask_noalloc

_DTYPES = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}

_c_i32, _c_i64, _c_p, _c_f, _c_sz = ctypes.c_int, ctypes.c_int64, ctypes.c_void_p, ctypes.c_float, ctypes.c_size_t

_SIGNATURES = {
    "actkv_error_string": (ctypes.c_char_p, [_c_i32]),
    "actkv_version": (ctypes.c_char_p, []),
    "actkv_action_scores": (_c_i32, [
        _c_p, _c_i32, _c_i64, _c_i64, _c_i64, _c_i64,            # q
        _c_p, _c_i32, _c_i64, _c_i64, _c_i64, _c_i64,            # kv
        _c_i64,                                                  # num_blocks
        _c_p, _c_i64, _c_i32,                                    # block_table, bt_sr, max_blocks
        _c_p,                                                    # seq_used
        _c_p, _c_i64, _c_i64, _c_i64,                            # lse
        _c_p, _c_i64, _c_i64, _c_i64, _c_i64,                    # out, strides, width
        _c_p, _c_p, _c_p,                                        # n_seen, n_valid, kv_len
        _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32,  # L R N Hq Hkv D bs
        _c_f, _c_p]),
    "actkv_copy_slots": (_c_i32, [_c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_i64, _c_p]),
    "actkv_keep_mask": (_c_i32, [
        _c_p, _c_i32, _c_i64, _c_i64, _c_i64,                    # scores
        _c_i32, _c_i32, _c_i32,                                  # L H R
        _c_p, _c_p, _c_p, _c_p, _c_i64,                          # seq_used budget prot_count prot_mask pm_sr
        _c_i32,                                                  # head_reduce
        _c_p, _c_i64, _c_p, _c_i64,                              # keep, keep_sr, bits, bits_sr
        _c_i32, _c_i32, _c_p, _c_sz, _c_p]),                     # bs, max_seq, ws, ws_bytes, stream
    "actkv_keep_mask_noalloc": (_c_i32, [
        _c_p, _c_i32, _c_i64, _c_i64, _c_i64,                    # scores
        _c_i32, _c_i32, _c_i32,                                  # L H R
        _c_p, _c_p, _c_p, _c_p, _c_i64,                          # seq_used budget prot_count prot_mask pm_sr
        _c_i32,                                                  # head_reduce
        _c_p, _c_i64, _c_p, _c_i64,                              # keep, keep_sr, bits, bits_sr
        _c_i32, _c_i32, _c_p]),                                  # bs, max_seq, stream
    "actkv_pack_keep": (_c_i32, [_c_p, _c_i64, _c_i32, _c_p, _c_i32, _c_p, _c_i64, _c_p, _c_i32, _c_p]),
    "actkv_compact": (_c_i32, [
        _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,            # kv planes sp ss row_bytes num_blocks
        _c_p, _c_i64, _c_i32, _c_p,                              # bits bits_sr R seq_used
        _c_p, _c_i64, _c_i32,                                    # block_table bt_sr bs
        _c_p, _c_i64, _c_p, _c_i64, _c_p, _c_p, _c_i64,          # perm pin_in pin_count pin_out
        _c_p, _c_i64, _c_p, _c_i64,                              # table_out freed
        _c_p, _c_p, _c_i64, _c_p,                                # src_out dst_out pairs_sr counts
        _c_i32, _c_i32, _c_i32, _c_p]),                          # do_copy max_seq max_kept stream
    "actkv_workspace_size": (_c_sz, [_c_i32, _c_i32, _c_i32]),
    "actkv_lrfu_update": (_c_i32, [
        _c_p, _c_i64, _c_i64, _c_i64, _c_i32, _c_i32, _c_i32,   # scores, strides, L H R
        _c_p, _c_p, _c_p, _c_i64, _c_p,                          # seq_used prot_count prot_mask pm_sr active
        _c_p, _c_i64, _c_i64,                                    # ks, strides
        _c_p, _c_i64, _c_i64,                                    # hit_out, strides
        _c_f, _c_f, _c_i32, _c_i32, _c_p, _c_sz, _c_p]),         # decay top_p reduce max_seq ws stream
    "actkv_lrfu_workspace_size": (_c_sz, [_c_i32, _c_i32, _c_i32]),
    "actkv_gather_tokens": (_c_i32, [_c_p, _c_i64, _c_i64, _c_p, _c_i64, _c_i64, _c_i32, _c_i32, _c_i32,
                                     _c_p, _c_i64, _c_p, _c_p]),
    "actkv_paged_attention": (_c_i32, [
        _c_p, _c_i32, _c_i64, _c_i64, _c_i64, _c_i64,            # q
        _c_p, _c_i32, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,    # kv, sl sv sb ss sh
        _c_i64,                                                  # num_blocks
        _c_p, _c_i64, _c_i32,                                    # block_table, bt_sr, max_blocks
        _c_p, _c_p, _c_p,                                        # seq_used n_valid kv_len
        _c_p, _c_i64, _c_i64, _c_i64, _c_i64,                    # out, strides
        _c_p, _c_i64, _c_i64, _c_i64,                            # lse, strides
        _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32,  # L R N Hq Hkv D bs
        _c_f, _c_p, _c_sz, _c_p]),                               # scale workspace bytes stream
    "actkv_paged_attention_workspace_size": (_c_sz, [_c_i32] * 8),
    "actkv_append": (_c_i32, [
        _c_p, _c_i32, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,  # kv, sl sv sb ss sh, num_blocks
        _c_p, _c_p, _c_i32,                                            # k v src_dtype
        _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,                # k strides, v strides
        _c_i32, _c_i32, _c_i32, _c_i32,                                # L Hkv D R
        _c_p, _c_p, _c_p, _c_i64,                                      # starts counts src_off total
        _c_p, _c_i64, _c_i32, _c_i32, _c_p, _c_p]),                    # table bt_sr mb bs bad stream
    "actkv_slot_map": (_c_i32, [_c_p, _c_i32, _c_i32, _c_i32, _c_i32, _c_p, _c_p]),
}

_lib = None


def lib() -> ctypes.CDLL:
    """Load the library once; raise if it has not been built."""
    global _lib, _glue_mod
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python actkv-open_amd/build_lib.py` "
                               "(the ActKV kernels have no CPU or Triton fallback)")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype, fn.argtypes = res, args
        # the HIP runtime the library links (torch's copy), reached through the library's own
        # dependency scope; the upload ring queues its host-to-device copies with it
        cp = handle.hipMemcpyAsync
        cp.restype, cp.argtypes = _c_i32, [_c_p, _c_p, _c_sz, _c_i32, _c_p]
        try:
            from . import _glue as g
        except ImportError as e:
            raise RuntimeError("the CPython call module actkv/_glue*.so is missing: build it with "
                               "`python actkv-open_amd/build_lib.py`") from e
        addr = lambda f: ctypes.cast(f, ctypes.c_void_p).value
        g.bind(addr(handle.actkv_action_scores), addr(handle.actkv_keep_mask), addr(handle.actkv_compact),
               addr(cp))
        _lib = handle
        _glue_mod = g
    return _lib


_glue_mod = None


def glue():
    """The bound _glue module: the scoring, keep-mask and compaction entry points and
    hipMemcpyAsync, called without ctypes' per-argument conversion (same arguments)."""
    if _glue_mod is None:
        lib()
    return _glue_mod


def available() -> bool:
    """True when the library is built and a ROCm GPU is visible."""
    return os.path.exists(LIB_PATH) and torch.cuda.is_available()


def debug() -> bool:
    """ACTKV_DEBUG=1 turns on host-side checks that read kernel reports back (they synchronise)."""
    return os.environ.get("ACTKV_DEBUG", "0") not in ("", "0")


def check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what} failed: {lib().actkv_error_string(rc).decode()}")


def dtype_code(dtype: torch.dtype) -> int:
    if dtype not in _DTYPES:
        raise TypeError(f"unsupported dtype {dtype}: the kernels take float32, float16 or bfloat16")
    return _DTYPES[dtype]


_GPU_DEVICES: dict = {}


def require_gpu(what: str, *tensors) -> torch.device:
    """All tensors must live on one ROCm GPU: the kernels have no CPU path.  (Device indices
    are compared as ints: building a torch.device per tensor costs a call's host time.)"""
    idx = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(f"{what} runs HIP kernels and needs tensors on a ROCm GPU, got {t.device}; "
                               "the *_ref functions are the CPU formulations")
        i = t.get_device()
        if idx is None:
            idx = i
        elif i != idx:
            raise RuntimeError(f"{what}: tensors on different devices (cuda:{idx}, cuda:{i})")
    if idx is None:
        return None
    dev = _GPU_DEVICES.get(idx)
    if dev is None:
        dev = _GPU_DEVICES[idx] = torch.device("cuda", idx)
    return dev


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


# torch's current-stream lookup without building a Stream object (several microseconds per
# call through torch.cuda.current_stream); the public route stays as the fallback.
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream(device: torch.device) -> int:
    """The hipStream_t of torch's current stream on `device` (the stream every launch uses)."""
    if _raw_stream is not None:
        return _raw_stream(device.index if device.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(device).cuda_stream


_workspaces: dict = {}
_HIP_MEMCPY_H2D = 1      # hipMemcpyHostToDevice


class _PinnedRing:
    """Host-to-device int32 uploads through one pinned staging buffer, used as a ring.

    Each upload copies into the next free span of the buffer, takes a fresh device tensor from
    torch's caching allocator and queues hipMemcpyAsync from the span into it (called directly:
    torch's own non-blocking copy also records a host-allocator event per call, which the ring
    makes unnecessary and which costs several microseconds).  The buffer is split in two halves: leaving a half records an event after its last
    copy, and coming back to that half waits for that event, so no span is rewritten before its
    copy has run.  One event per half-buffer of uploads (thousands of calls), instead of one per
    upload (an event record costs a current-stream lookup, several microseconds).  Uploads larger
    than half the buffer are copied synchronously from pageable memory."""

    SIZE = 1 << 18          # int32 entries (1 MiB)

    def __init__(self):
        self.buf = None
        self.np = None
        self.half = 0                    # the half the next span is taken from
        self.off = 0                     # the next free entry (inside that half)
        self.events = [None, None]       # per half: event after its last copy, or "sync"
        self.streams = [set(), set()]    # per half: the streams its copies were queued on

    def upload_i32(self, values, device: torch.device) -> torch.Tensor:
        arr = np.asarray(values, dtype=np.int32).reshape(-1)
        n = arr.size
        half = self.SIZE // 2
        if n > half:
            return torch.from_numpy(arr.copy()).to(device)
        if self.buf is None:
            self.buf = torch.empty(self.SIZE, dtype=torch.int32, pin_memory=True)
            self.np = self.buf.numpy()
            # touch every page now: a first write to a page of the fresh buffer costs a fault
            # of several microseconds, which would otherwise land on the uploads of the first
            # pass through the ring
            self.np[:] = 0
        # the current half is tracked, not derived from the offset: a half filled to its last
        # entry leaves the offset on the next half's first entry (or one past the buffer), and
        # the next upload must still go through the change of halves below
        h = self.half
        cur = stream(device)
        if self.off + n > (h + 1) * half:
            # leave half h (its copies are all queued): an event on the stream that queued them
            # covers them; copies queued on several streams are covered by a device sync later
            if self.streams[h] <= {cur}:
                ev = torch.cuda.Event()
                ev.record()
                self.events[h] = ev
            else:
                self.events[h] = "sync"
            h = 1 - h
            self.half = h
            self.off = h * half
            if self.events[h] == "sync":
                torch.cuda.synchronize(device)
            elif self.events[h] is not None:
                self.events[h].synchronize()
            self.events[h] = None
            self.streams[h] = set()
        self.streams[h].add(cur)
        self.np[self.off:self.off + n] = arr
        out = torch.empty(n, dtype=torch.int32, device=device)
        if n:
            rc = glue().memcpy_async(out.data_ptr(), self.buf.data_ptr() + 4 * self.off, 4 * n,
                                      _HIP_MEMCPY_H2D, cur)
            if rc != 0:
                raise RuntimeError(f"hipMemcpyAsync (host to device, {4 * n} bytes) failed with HIP error {rc}")
        self.off += n
        return out


_rings: dict = {}


def upload_i32(values, device: torch.device) -> torch.Tensor:
    """Host ints -> a new device int32 tensor, asynchronously on the current stream."""
    ring = _rings.get(device)
    if ring is None:
        ring = _rings[device] = _PinnedRing()
    return ring.upload_i32(values, device)


def scratch(device: torch.device, key, nbytes: int) -> torch.Tensor:
    """A cached uint8 device buffer of at least nbytes for `key`, grown on demand (contents
    undefined).  Calls sharing it are ordered on the current stream."""
    full = (device, key)
    buf = _workspaces.get(full)
    if buf is None or buf.numel() < nbytes:
        # grown geometrically: a workload whose sizes creep up reallocates a few times, not
        # on every call (a device allocation can cost milliseconds)
        old = 0 if buf is None else buf.numel()
        buf = torch.empty(max(int(nbytes), 2 * old, 1 << 16), dtype=torch.uint8, device=device)
        _workspaces[full] = buf
    return buf


_ws_sizes: dict = {}


def workspace(device: torch.device, kind: int, r: int, max_seq: int) -> torch.Tensor:
    """Cached per (device, kind) and grown on demand; the kernels need no initialised
    contents.  Calls sharing it are ordered on the current stream."""
    need = _ws_sizes.get((kind, r, max_seq))
    if need is None:                # the size is a pure function of its arguments
        if len(_ws_sizes) > 4096:
            _ws_sizes.clear()
        need = _ws_sizes[(kind, r, max_seq)] = int(lib().actkv_workspace_size(kind, r, max_seq))
    key = (device, kind)
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < need:
        old = 0 if ws is None else ws.numel()
        ws = torch.empty(max(need, 2 * old, 1 << 16), dtype=torch.uint8, device=device)
        _workspaces[key] = ws
    return ws

"""Streaming safetensors I/O for the model loop (the reference loads the
whole model with ``load_file`` and writes it with one ``save_file``,
converter/pipeline.py:268, 1116-1121).

* ``SafetensorsIndex`` parses a file's header: tensors in data order, which
  is the order ``load_file`` returns them in (the reference's loop order).
* ``Prefetcher`` reads the next layers' bytes on a host thread into pinned
  buffers (each large tensor split over several reader threads: one
  thread's copies out of the page cache run at well under the host's
  memory bandwidth) and copies them to the GPU on a copy stream while the
  current layer computes.
* ``StreamWriter`` writes outputs as they are produced: device results are
  copied to pooled pinned chunks on a D2H stream, host threads write them at
  the offsets assigned on arrival (positional writes, in parallel), and
  tensors passed through unchanged are copied file to file.  The
  header goes into a region reserved at the start and padded with spaces
  (the safetensors format allows a space-padded header), so no tensor is
  held until the end.  The file is written under a temporary name and
  renamed when complete: an aborted run leaves no output.
"""

from __future__ import annotations

import concurrent.futures as cf
import json
import os
import queue
import struct
import threading

import torch

ST_TO_TORCH = {
    "F64": torch.float64, "F32": torch.float32, "F16": torch.float16, "BF16": torch.bfloat16,
    "I64": torch.int64, "I32": torch.int32, "I16": torch.int16, "I8": torch.int8, "U8": torch.uint8,
    "BOOL": torch.bool,
}
TORCH_TO_ST = {v: k for k, v in ST_TO_TORCH.items()}


class SafetensorsIndex:
    """Header of a safetensors file: name -> (dtype, shape, begin, end) in
    data order; absolute byte offsets."""

    def __init__(self, path: str):
        self.path = path
        with open(path, "rb") as f:
            n = struct.unpack("<Q", f.read(8))[0]
            header = json.loads(f.read(n))
        self.metadata = header.pop("__metadata__", None)
        base = 8 + n
        items = sorted(header.items(), key=lambda kv: kv[1]["data_offsets"][0])
        self.entries = {}
        for name, e in items:
            b, end = e["data_offsets"]
            if e["dtype"] not in ST_TO_TORCH:
                raise ValueError(f"{path}: unsupported dtype {e['dtype']} for {name}")
            self.entries[name] = (ST_TO_TORCH[e["dtype"]], tuple(e["shape"]), base + b, base + end)

    def names(self) -> list[str]:
        return list(self.entries)

    def nbytes(self, name: str) -> int:
        _, _, b, e = self.entries[name]
        return e - b

    def read(self, name: str, out: torch.Tensor | None = None, pool: cf.Executor | None = None,
             parts: int = 1) -> torch.Tensor:
        """The tensor as a CPU tensor (into `out`'s storage when given: a
        uint8 buffer of at least nbytes, e.g. pinned).  With `pool`, a
        tensor of at least READ_SPLIT bytes is read as up to `parts`
        positional reads of consecutive byte ranges on the pool's threads."""
        dtype, shape, b, e = self.entries[name]
        n = e - b
        buf = out[:n] if out is not None else torch.empty(n, dtype=torch.uint8)
        mv = memoryview(buf.numpy())
        fd = os.open(self.path, os.O_RDONLY)
        try:
            k = max(1, min(parts, n // READ_SPLIT)) if pool is not None else 1
            step = -(-n // k)
            spans = [(o, min(n, o + step)) for o in range(0, n, step)] if n else []
            if k == 1:
                for lo, hi in spans:
                    _pread_into(fd, mv[lo:hi], b + lo, self.path, name)
            else:
                futs = [pool.submit(_pread_into, fd, mv[lo:hi], b + lo, self.path, name) for lo, hi in spans]
                for f in futs:
                    f.result()
        finally:
            os.close(fd)
        t = buf.view(dtype) if n else torch.empty(0, dtype=dtype)
        return t.reshape(shape)


READ_SPLIT = 8 << 20      # smallest byte range a parallel read hands to one thread


def _pread_into(fd: int, mv: memoryview, pos: int, path: str, name: str) -> None:
    got = 0
    while got < len(mv):
        r = os.preadv(fd, [mv[got:]], pos + got)
        if not r:
            raise IOError(f"{path}: short read of {name}")
        got += r


class PinnedPool:
    """Process-wide pinned host buffers, allocated once and reused: pinned
    allocation costs far more than the copies it serves."""

    def __init__(self):
        self._lock = threading.Lock()
        self._free: dict[int, list[torch.Tensor]] = {}

    def take(self, nbytes: int) -> torch.Tensor:
        size = 1 << max(20, (max(nbytes, 1) - 1).bit_length())      # power-of-2 size classes from 1 MiB
        with self._lock:
            lst = self._free.get(size)
            if lst:
                return lst.pop()
        return torch.empty(size, dtype=torch.uint8, pin_memory=True)

    def give(self, buf: torch.Tensor):
        with self._lock:
            self._free.setdefault(buf.numel(), []).append(buf)


POOL = PinnedPool()
CHUNK = 32 << 20          # D2H staging chunk (bytes)


class Prefetcher:
    """Reads `names` in order on a host thread into pinned buffers (`depth`
    of them) and copies each to the GPU on a copy stream one layer ahead:
    get(name) returns layer k and starts layer k + 1's copy, which then
    overlaps the caller's work on layer k.  Names must be requested in
    order."""

    def __init__(self, index: SafetensorsIndex, names: list[str], device, depth: int = 2, readers: int = 8):
        self.index = index
        self.readers = readers
        self.pool = cf.ThreadPoolExecutor(max_workers=readers) if readers > 1 else None
        self.names = list(names)
        self.device = device
        cap = max([index.nbytes(n) for n in self.names] + [1])
        self.bufs = [POOL.take(cap) for _ in range(depth)]
        self.free: queue.Queue = queue.Queue()
        for b in self.bufs:
            self.free.put(b)
        self.ready: queue.Queue = queue.Queue()
        self.stream = torch.cuda.Stream(device=device)
        self.inflight: dict[str, tuple] = {}
        self.started = 0
        self.error: BaseException | None = None
        self.thread = threading.Thread(target=self._run, daemon=True)
        self.thread.start()

    def _run(self):
        try:
            for name in self.names:
                buf = self.free.get()
                if buf is None:
                    return
                t = self.index.read(name, buf, self.pool, self.readers)
                self.ready.put((name, buf, t))
        except BaseException as e:  # surfaced to the consumer
            self.error = e
            self.ready.put(None)

    def _start_next(self):
        if self.started >= len(self.names):
            return
        item = self.ready.get()
        if item is None:
            raise RuntimeError(f"reading {self.index.path} failed: {self.error}") from self.error
        name, buf, t = item
        self.started += 1
        with torch.cuda.stream(self.stream):
            g = torch.empty(t.shape, dtype=t.dtype, device=self.device)
            g.copy_(t, non_blocking=True)
            ev = torch.cuda.Event()
            ev.record(self.stream)
        self.inflight[name] = (g, buf, ev)

    def get(self, name: str) -> torch.Tensor:
        if name not in self.inflight:
            self._start_next()
        if name not in self.inflight:
            raise KeyError(f"{name} requested out of order")
        g, buf, ev = self.inflight.pop(name)
        cur = torch.cuda.current_stream(self.device)
        cur.wait_event(ev)
        g.record_stream(cur)
        ev.synchronize()          # its pinned buffer can be refilled
        self.free.put(buf)
        self._start_next()
        return g

    def close(self):
        for _ in range(len(self.bufs) + 2):
            self.free.put(None)
        self.thread.join()
        for g, buf, ev in self.inflight.values():
            ev.synchronize()
        self.inflight.clear()
        if self.pool is not None:
            self.pool.shutdown(wait=True)
            self.pool = None
        for b in self.bufs:
            POOL.give(b)
        self.bufs = []


class StreamWriter:
    """Writes tensors into a safetensors file as they come, with `workers`
    host threads issuing positional writes at the offsets assigned on
    arrival; the header goes into the reserved region at close."""

    def __init__(self, path: str, reserve: int, device=None, workers: int = 4):
        self.path = path
        self.tmp = path + ".partial"
        self.reserve = max(int(reserve), 64)
        self.fd = os.open(self.tmp, os.O_RDWR | os.O_CREAT | os.O_TRUNC, 0o644)
        self.base = 8 + self.reserve
        self.offset = 0
        self.header: dict[str, dict] = {}
        self.jobs: queue.Queue = queue.Queue(maxsize=16)
        self.error: BaseException | None = None
        self.device = device
        self.stream = torch.cuda.Stream(device=device) if device is not None else None
        self.threads = [threading.Thread(target=self._run, daemon=True) for _ in range(workers)]
        for t in self.threads:
            t.start()
        self.closed = False

    def _record(self, name, dtype, shape, n):
        if name in self.header:
            raise ValueError(f"tensor {name} written twice")
        off = self.offset
        self.header[name] = {"dtype": TORCH_TO_ST[dtype], "shape": list(shape), "data_offsets": [off, off + n]}
        self.offset += n
        return self.base + off

    def _pwrite(self, data, pos):
        mv = memoryview(data)
        while len(mv):
            k = os.pwrite(self.fd, mv, pos)
            mv = mv[k:]
            pos += k

    def _run(self):
        while True:
            job = self.jobs.get()
            if job is None:
                return
            try:
                kind = job[0]
                if kind == "host":
                    _, data, pos = job
                    self._pwrite(data.numpy(), pos)
                elif kind == "dev":
                    _, ev, buf, n, pos = job
                    ev.synchronize()
                    self._pwrite(buf[:n].numpy(), pos)
                    POOL.give(buf)
                elif kind == "copy":
                    _, src_path, b, n, pos = job
                    with open(src_path, "rb", buffering=0) as src:
                        done = 0
                        while done < n:
                            chunk = os.pread(src.fileno(), min(n - done, CHUNK), b + done)
                            if not chunk:
                                raise IOError(f"{src_path}: short read")
                            self._pwrite(chunk, pos + done)
                            done += len(chunk)
            except BaseException as e:
                self.error = e

    def _put(self, job):
        if self.error is not None:
            raise RuntimeError(f"stream writer failed: {self.error}") from self.error
        self.jobs.put(job)

    def add_host(self, name: str, t: torch.Tensor):
        t = t.contiguous()
        data = t.reshape(-1).view(torch.uint8) if t.numel() else torch.empty(0, dtype=torch.uint8)
        pos = self._record(name, t.dtype, t.shape, data.numel())
        if data.numel():
            self._put(("host", data, pos))

    def add_file_copy(self, name: str, index: SafetensorsIndex):
        dtype, shape, b, e = index.entries[name]
        pos = self._record(name, dtype, shape, e - b)
        if e > b:
            self._put(("copy", index.path, b, e - b, pos))

    def add_device(self, name: str, t: torch.Tensor):
        """Copy a GPU tensor to pooled pinned chunks on the D2H stream (after
        the current stream's work on it); the writers append each chunk
        when its copy is done."""
        t = t.contiguous()
        n = t.numel() * t.element_size()
        pos = self._record(name, t.dtype, t.shape, n)
        if n == 0:
            return
        flat = t.reshape(-1).view(torch.uint8)
        self.stream.wait_stream(torch.cuda.current_stream(t.device))
        for c0 in range(0, n, CHUNK):
            k = min(CHUNK, n - c0)
            buf = POOL.take(k)
            with torch.cuda.stream(self.stream):
                buf[:k].copy_(flat[c0:c0 + k], non_blocking=True)
                ev = torch.cuda.Event()
                ev.record(self.stream)
            self._put(("dev", ev, buf, k, pos + c0))
        t.record_stream(self.stream)

    def _stop(self):
        for _ in self.threads:
            self.jobs.put(None)
        for t in self.threads:
            t.join()

    def close(self, metadata: dict | None):
        self._stop()
        self.closed = True
        if self.error is not None:
            self.abort()
            raise RuntimeError(f"stream writer failed: {self.error}") from self.error
        hdr = dict(self.header)
        if metadata:
            hdr = {"__metadata__": metadata, **hdr}
        blob = json.dumps(hdr, separators=(",", ":")).encode("utf-8")
        if len(blob) > self.reserve:
            # header larger than reserved: rewrite with the data shifted
            os.close(self.fd)
            self._rewrite(blob)
        else:
            blob = blob + b" " * (self.reserve - len(blob))
            self._pwrite(struct.pack("<Q", len(blob)) + blob, 0)
            os.close(self.fd)
        # renaming over an existing file makes some file systems flush the new
        # one first; the old output is removed only now that the new is whole
        if os.path.exists(self.path):
            os.remove(self.path)
        os.replace(self.tmp, self.path)

    def _rewrite(self, blob: bytes):
        pad = (-len(blob)) % 8
        blob = blob + b" " * pad
        fixed = self.tmp + ".2"
        with open(self.tmp, "rb") as src, open(fixed, "wb") as dst:
            dst.write(struct.pack("<Q", len(blob)))
            dst.write(blob)
            src.seek(self.base)
            while True:
                chunk = src.read(64 << 20)
                if not chunk:
                    break
                dst.write(chunk)
        os.replace(fixed, self.tmp)

    def abort(self):
        if not self.closed:
            self.closed = True
            try:
                while True:
                    self.jobs.get_nowait()
            except queue.Empty:
                pass
            self._stop()
            try:
                os.close(self.fd)
            except OSError:
                pass
        if os.path.exists(self.tmp):
            os.remove(self.tmp)


def header_reserve(index: SafetensorsIndex, metadata: dict) -> int:
    """Bytes to reserve for the output header: up to six entries per input
    tensor (weights, scale, zero-point, permutation, two ComfyUI blobs)."""
    per = sum(6 * (len(n) + 160) for n in index.names())
    return 4096 + per + 2 * len(json.dumps(metadata))

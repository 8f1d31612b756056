"""dattri-llm's on-disk gradient store, read into the scoring loop through
pinned host buffers and asynchronous host-to-device copies.

Format (the reference's ``disk_format="memmap"``, ``gradient/storage_manager.py:46-56``,
written by ``:620-694`` and read by ``:697-763``; index ``:159-299``, ``:1062-1135``)::

    save_dir/index_meta.json   {"format": 2, "sample_id_key": ..., "gradient_accumulation_steps": 1}
    save_dir/index.jsonl       one line per saved group:
                               {"file": "batch_000000.mmap", "records": [{"idx", "step", "hashes"}]}
    save_dir/batch_NNNNNN.mmap.bin   every layer's raw tensor bytes, each part 8-byte aligned
    save_dir/batch_NNNNNN.mmap.meta  torch.save({"format": 2, "records": [...]}), primitives only:
                               per record step, input_hash, sample_id_key, representation,
                               layer_types, indexing and per layer {"kind": "dense"|"factorized",
                               "parts": {name: {"byte_off", "nbytes", "shape", "dtype"}}, ...}

Under ``torch.distributed`` the reference writes ``save_dir/rank_N/``; the
reader merges every rank's index, with paths relative to ``save_dir``.  The
meta is loaded with ``torch.load(weights_only=True)`` and the payload is a
private memory map, so reading executes nothing from the files; pickled
``.pt`` groups (the reference's ``disk_format="pickle"``) are refused.

:class:`PinnedBlockSource` is the scoring loop's view of a store (the
reference's ``DiskGradientSource`` over ``GradientFileMultiStepDataset``,
``gradient/streaming.py:95-180``, ``gradient/datasets.py:100-249``): one
``(step, Gradient, hashes)`` block per (file, step), in the store's file
order.  A reader thread reads each file's bytes straight into one pinned host
buffer (parallel ``preadv``); the caller's thread copies it to the GPU on a
copy stream one file ahead, so the next file's transfer overlaps the kernels
scoring the current one, and the records are device views at their stored
offsets (8-byte aligned, so every dtype view is legal).
:class:`AsyncGradientWriter` is the write side (``gradient/async_writer.py``):
groups are copied off the GPU on the writer's own stream and written in
submission order by one thread.
"""

from __future__ import annotations

import json
import os
import queue
import threading
import warnings
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import numpy as np
import torch

from dattri_llm_amd.gradient.gradient import Factorized, Gradient, GradientRecord, base_layer_name
from dattri_llm_amd.gradient.ops.types import PARAM_GRAD_TYPES

MEMMAP_FORMAT = 2
INDEX_FORMAT = 2
INDEX_LOG_FILE = "index.jsonl"
INDEX_META_FILE = "index_meta.json"

_DTYPE_BY_NAME = {str(v).removeprefix("torch."): v for v in vars(torch).values() if isinstance(v, torch.dtype)}


def _dtype_name(dtype: torch.dtype) -> str:
    return str(dtype).removeprefix("torch.")


def _dtype_from_name(name: str) -> torch.dtype:
    try:
        return _DTYPE_BY_NAME[name]
    except KeyError:
        raise ValueError(f"Unknown tensor dtype {name!r} in memmap metadata.") from None


# ---------------------------------------------------------------------------
# group codec: one layer value <-> the format's (kind, tensor parts, extras),
# shared by the writer and the reader
# ---------------------------------------------------------------------------

_PART_ALIGN = 8  # every part starts 8-byte aligned, so any dtype can be viewed at its offset


def _split_layer(value) -> tuple[str, dict[str, torch.Tensor], dict]:
    """A layer as the format stores it: its kind, its tensor parts by name and
    the non-tensor fields kept beside them in the meta."""
    if isinstance(value, Factorized):
        parts = {"activation": value.activation, "pre_activation_grad": value.pre_activation_grad}
        return "factorized", parts, {"module_kwargs": value.module_kwargs, "batch_first": value.batch_first}
    return "dense", {"data": value}, {}


def _join_layer(kind: str, parts: dict[str, torch.Tensor], fields: dict):
    """The layer value :func:`_split_layer` took apart."""
    if kind == "factorized":
        return Factorized(parts["activation"], parts["pre_activation_grad"],
                          module_kwargs=fields["module_kwargs"], batch_first=fields["batch_first"])
    return parts["data"]


class _BinLayout:
    """The ``.bin`` of one group, planned before it is written: parts are
    placed in record, layer, part order, each at the next aligned offset, and
    the file ends on an aligned boundary."""

    def __init__(self) -> None:
        self.parts: list[tuple[int, torch.Tensor]] = []
        self.size = 0

    def place(self, tensor: torch.Tensor) -> dict:
        host = tensor.detach().to("cpu").contiguous()
        nbytes = host.numel() * host.element_size()
        offset = self.size
        self.parts.append((offset, host))
        end = offset + nbytes
        self.size = end + (-end) % _PART_ALIGN
        return {"byte_off": offset, "nbytes": nbytes, "shape": list(host.shape), "dtype": _dtype_name(host.dtype)}

    def write(self, path: Path) -> None:
        with open(path, "wb") as f:
            pos = 0
            for offset, host in self.parts:
                if offset > pos:
                    f.write(bytes(offset - pos))
                if host.numel():
                    f.write(memoryview(host.view(torch.uint8).reshape(-1).numpy()))
                pos = offset + host.numel() * host.element_size()
            if self.size > pos:
                f.write(bytes(self.size - pos))


def _record_meta(record: GradientRecord, layout: _BinLayout) -> dict:
    """A record's meta entry, its tensors placed in ``layout``."""
    g = record.gradient
    layers = {}
    for name, value in g.data.items():
        kind, parts, fields = _split_layer(value)
        layers[name] = {"kind": kind, "parts": {p: layout.place(t) for p, t in parts.items()}, **fields}
    return {"step": record.step, "input_hash": record.input_hash, "sample_id_key": record.sample_id_key,
            "representation": dict(g.representation), "layer_types": dict(g.layer_types),
            "indexing": dict(g.indexing), "layers": layers}


class GradientStore:
    """Index, reader and writer of a memmap gradient store (one process, one rank)."""

    def __init__(self, save_dir: str | Path) -> None:
        self.root = Path(save_dir)
        self._index: dict[str, list[dict]] = {}
        self._sample_id_key = None
        self._next_batch_id: int | None = None
        self._metas: dict[str, dict] = {}  # parsed group metas (a saved group never changes)
        if self.root.exists():
            self._read_index()

    # -- index -------------------------------------------------------------

    def _read_index(self) -> None:
        dirs = [self.root] + sorted(p for p in self.root.glob("rank_*") if p.is_dir())
        for d in dirs:
            meta = d / INDEX_META_FILE
            if meta.exists():
                info = json.loads(meta.read_text())
                if info.get("format") != INDEX_FORMAT:
                    raise ValueError(f"{meta} has index format {info.get('format')!r}, expected {INDEX_FORMAT}")
                self._sample_id_key = info.get("sample_id_key", self._sample_id_key)
            log = d / INDEX_LOG_FILE
            if not log.exists():
                continue
            for line in log.read_text().splitlines():
                if not line.strip():
                    continue
                payload = json.loads(line)
                for rec in payload["records"]:
                    for sample_idx, h in enumerate(rec["hashes"]):
                        entry = {"file": payload["file"], "idx": rec["idx"], "step": rec["step"],
                                 "sample_idx": sample_idx}
                        entries = self._index.setdefault(h, [])
                        if entry not in entries:
                            entries.append(entry)

    @property
    def index(self) -> dict[str, list[dict]]:
        return self._index

    @property
    def sample_id_key(self):
        return self._sample_id_key

    def available_steps(self) -> list[int]:
        return sorted({e["step"] for entries in self._index.values() for e in entries})

    def iter_steps(self, steps) -> list[tuple[str, dict[int, list[int]]]]:
        """``(file, {step: record idxs})`` per file holding the steps, by file name
        (storage_manager.py:1071-1109)."""
        wanted = {steps} if isinstance(steps, int) else set(steps)
        by_file: dict[str, dict[int, set[int]]] = {}
        for entries in self._index.values():
            for e in entries:
                if e["step"] in wanted:
                    by_file.setdefault(e["file"], {}).setdefault(e["step"], set()).add(e["idx"])
        return [(f, {s: sorted(ix) for s, ix in sorted(by_file[f].items())}) for f in sorted(by_file)]

    # -- reading -----------------------------------------------------------

    def read_meta(self, file_rel: str) -> dict:
        """A group's meta (primitives only, ``torch.load(weights_only=True)``),
        parsed once per store object."""
        cached = self._metas.get(file_rel)
        if cached is not None:
            return cached
        if not file_rel.endswith(".mmap"):
            raise NotImplementedError(
                f"{file_rel}: pickled gradient groups are not read (loading them would execute pickled "
                "code); collect the store with disk_format='memmap'."
            )
        handle = self.root / file_rel
        payload = torch.load(Path(f"{handle}.meta"), weights_only=True)
        if not isinstance(payload, dict) or payload.get("format") != MEMMAP_FORMAT:
            found = payload.get("format") if isinstance(payload, dict) else "pre-v2"
            raise ValueError(
                f"{handle.name} was written in memmap format {found!r}, but this version reads format "
                f"{MEMMAP_FORMAT}. Re-collect the store; the byte offsets are not compatible."
            )
        self._metas[file_rel] = payload
        return payload

    def bin_nbytes(self, file_rel: str) -> int:
        return Path(f"{self.root / file_rel}.bin").stat().st_size

    def read_bin_into(self, file_rel: str, out: torch.Tensor, pool: ThreadPoolExecutor | None = None) -> None:
        """Read a group's ``.bin`` into ``out`` (a CPU uint8 tensor of its size,
        e.g. pinned memory) with parallel ``preadv`` calls."""
        n = out.numel()
        if n == 0:
            return
        view = memoryview(out.numpy())
        fd = os.open(f"{self.root / file_rel}.bin", os.O_RDONLY)
        try:
            chunk = max(1 << 22, -(-n // 8))

            def work(start: int) -> None:
                pos, end = start, min(n, start + chunk)
                while pos < end:
                    got = os.preadv(fd, [view[pos:end]], pos)
                    if got <= 0:
                        raise EOFError(f"{file_rel}.bin ended at byte {pos} of {n}")
                    pos += got

            starts = range(0, n, chunk)
            if pool is None or len(starts) == 1:
                for st in starts:
                    work(st)
            else:
                list(pool.map(work, starts))
        finally:
            os.close(fd)

    def records_from(self, payload: dict, buffer: torch.Tensor, file_rel: str = "") -> list[GradientRecord]:
        """The records of a group as views into ``buffer``, the group's ``.bin``
        bytes (a memory map, a pinned host buffer or a device buffer)."""

        def view(spec: dict) -> torch.Tensor:
            dtype, shape = _dtype_from_name(spec["dtype"]), tuple(spec["shape"])
            off, n = spec["byte_off"], spec["nbytes"]
            if n == 0:
                return torch.empty(shape, dtype=dtype, device=buffer.device)
            if off % _PART_ALIGN or off + n > buffer.numel():
                raise ValueError(f"{file_rel}: part at byte {off} (+{n}) is misaligned or past the file")
            return buffer[off:off + n].view(dtype).reshape(shape)

        def gradient(meta: dict) -> Gradient:
            data = {name: _join_layer(layer["kind"], {p: view(spec) for p, spec in layer["parts"].items()}, layer)
                    for name, layer in meta["layers"].items()}
            return Gradient(meta["representation"], data, meta["layer_types"], meta["indexing"],
                            validate_on_init=False)

        return [GradientRecord(m["step"], m["input_hash"], gradient(m), m["sample_id_key"])
                for m in payload["records"]]

    def load_records(self, file_rel: str) -> list[GradientRecord]:
        """The records of one group as CPU tensors viewing a private map of the file."""
        payload = self.read_meta(file_rel)
        total = self.bin_nbytes(file_rel)
        bin_path = f"{self.root / file_rel}.bin"
        buffer = (torch.from_numpy(np.memmap(bin_path, dtype=np.uint8, mode="c", shape=(total,)))
                  if total else torch.empty(0, dtype=torch.uint8))
        return self.records_from(payload, buffer, file_rel)

    # -- writing -----------------------------------------------------------

    def save_bulk(self, records: list[GradientRecord]) -> str:
        """Write one group (CPU tensors) as ``batch_NNNNNN.mmap`` and append its
        index line (write-then-index, storage_manager.py:491-521, :620-694)."""
        self.root.mkdir(parents=True, exist_ok=True)
        if self._next_batch_id is None:
            ids = [int(p.name[6:12]) for p in self.root.glob("batch_*.mmap.meta") if p.name[6:12].isdigit()]
            self._next_batch_id = max(ids) + 1 if ids else 0
        base = f"batch_{self._next_batch_id:06d}.mmap"
        self._next_batch_id += 1
        layout = _BinLayout()
        meta_records = [_record_meta(rec, layout) for rec in records]
        layout.write(self.root / f"{base}.bin")
        torch.save({"format": MEMMAP_FORMAT, "records": meta_records}, self.root / f"{base}.meta")
        meta_file = self.root / INDEX_META_FILE
        if not meta_file.exists():
            meta_file.write_text(json.dumps({"format": INDEX_FORMAT, "sample_id_key": records[0].sample_id_key
                                             if records else None, "gradient_accumulation_steps": 1}))
        line = {"file": base, "records": [
            {"idx": i, "step": r.step, "hashes": r.input_hash if isinstance(r.input_hash, list) else [r.input_hash]}
            for i, r in enumerate(records)]}
        with open(self.root / INDEX_LOG_FILE, "a") as log:
            log.write(json.dumps(line) + "\n")
        for entry in line["records"]:
            for sample_idx, h in enumerate(entry["hashes"]):
                self._index.setdefault(h, []).append({"file": base, "idx": entry["idx"], "step": entry["step"],
                                                      "sample_idx": sample_idx})
        return base


# ---------------------------------------------------------------------------
# blocks: records of one (file, step) joined along the batch axis
# ---------------------------------------------------------------------------


def _cat_layer(values):
    first = values[0]
    if isinstance(first, Factorized):
        dim = 0 if first.batch_first else 1
        return Factorized(torch.cat([v.activation for v in values], dim), torch.cat([v.pre_activation_grad
                          for v in values], dim), module_kwargs=first.module_kwargs, batch_first=first.batch_first)
    return values[0] if len(values) == 1 else torch.cat(values, 0)


def records_to_block(records, idxs, layer_name=None):
    """One ``(Gradient, hashes)`` block from the records ``idxs`` of a group
    (datasets.py:40-97).  A requested layer name also selects its invocation
    layers (``"lin"`` pulls in ``"lin@2"``); batch-level ``param_grad`` layers
    have no per-sample rows and are left out with a warning."""
    grads, hashes, dropped = [], [], set()
    for i in idxs:
        rec = records[i]
        g = rec.gradient
        names = g.layer_names if layer_name is None else set(layer_name)
        missing = names - g.layer_names
        if missing:
            raise KeyError(f"Unknown layers: {sorted(missing)}")
        if layer_name is not None:
            names = names | {n for n in g.layer_names if base_layer_name(n) in names}
        batch_level = {n for n in names if g.layer_types[n] == PARAM_GRAD_TYPES}
        dropped |= batch_level
        names = names - batch_level
        if not names:
            raise ValueError("No per-sample gradient layers remain once the batch-level param_grad layers "
                             f"{sorted(batch_level)} are left out.")
        grads.append((g, sorted(names)))
        h = rec.input_hash
        hashes.extend(h if isinstance(h, list) else [h])
    if dropped:
        warnings.warn(f"Skipping batch-level param_grad layers during per-sample attribution: {sorted(dropped)}.",
                      stacklevel=3)
    if not grads:
        raise RuntimeError("no records selected")
    g0, names = grads[0]
    data = {n: _cat_layer([g.data[n] for g, _ in grads]) for n in names}
    block = Gradient({n: g0.representation[n] for n in names}, data, {n: g0.layer_types[n] for n in names},
                     {n: g0.indexing.get(n, "batch") for n in names}, validate_on_init=False)
    if block.batch_size != len(hashes):
        raise RuntimeError(f"block batch size ({block.batch_size}) disagrees with hash count ({len(hashes)})")
    return block, hashes


def _map_tensors(block: Gradient, fn) -> Gradient:
    data = {}
    for n, v in block.data.items():
        if isinstance(v, Factorized):
            data[n] = Factorized(fn(v.activation), fn(v.pre_activation_grad), module_kwargs=v.module_kwargs,
                                 batch_first=v.batch_first)
        else:
            data[n] = fn(v)
    return Gradient(dict(block.representation), data, dict(block.layer_types), dict(block.indexing),
                    validate_on_init=False)


class PinnedBlockSource:
    """``(step, Gradient, hashes)`` blocks of a store, delivered on ``device``
    (a ROCm device through pinned buffers and a copy stream; the host, as
    plain host tensors).

    ``steps``: the stored steps to read (``None``: all); ``layer_name``: a layer
    filter; ``prefetch``: host blocks the reader thread keeps ready."""

    reusable = True

    def __init__(self, store: GradientStore | str | Path, *, device="cuda", steps=None, layer_name=None,
                 prefetch: int = 2) -> None:
        self.store = store if isinstance(store, GradientStore) else GradientStore(store)
        available = self.store.available_steps()
        if steps is None:
            self.steps = available
        else:
            wanted = set(steps)
            self.steps = [s for s in available if s in wanted]
            if not self.steps:
                raise ValueError(f"None of the requested steps {sorted(wanted)} are present in the gradients; "
                                 f"available steps: {available}.")
        self.layer_name = None if layer_name is None else ([layer_name] if isinstance(layer_name, str)
                                                           else list(layer_name))
        self.device = torch.device(device)
        self.prefetch = max(1, int(prefetch))
        self.h2d_bytes = 0

    def __len__(self) -> int:
        return sum(len(by_step) for _f, by_step in self.store.iter_steps(self.steps))

    @staticmethod
    def _put(out: queue.Queue, item, stop: threading.Event) -> bool:
        """Hand ``item`` to the consumer; False once the consumer has stopped
        (so a reader never blocks on a full queue nobody drains)."""
        while not stop.is_set():
            try:
                out.put(item, timeout=0.1)
                return True
            except queue.Full:
                continue
        return False

    def _host_files(self, out: queue.Queue, stop: threading.Event) -> None:
        """Reader thread: each file's meta and its bytes in a pinned buffer,
        then ``None``; an exception is handed over in place of the rest."""
        try:
            with ThreadPoolExecutor(max_workers=8) as pool:
                for file_rel, by_step in self.store.iter_steps(self.steps):
                    if stop.is_set():
                        return
                    payload = self.store.read_meta(file_rel)
                    host = torch.empty(self.store.bin_nbytes(file_rel), dtype=torch.uint8, pin_memory=True)
                    self.store.read_bin_into(file_rel, host, pool)
                    if not self._put(out, (file_rel, by_step, payload, host), stop):
                        return
            self._put(out, None, stop)
        except BaseException as exc:  # noqa: BLE001 - handed to the consumer
            self._put(out, exc, stop)

    def _host_blocks(self):
        """The blocks in host memory, one file at a time with no reader thread
        or copy stream: the same records, for a source whose device is the
        host."""
        for file_rel, by_step in self.store.iter_steps(self.steps):
            payload = self.store.read_meta(file_rel)
            host = torch.empty(self.store.bin_nbytes(file_rel), dtype=torch.uint8)
            self.store.read_bin_into(file_rel, host)
            records = self.store.records_from(payload, host, file_rel)
            for step, idxs in by_step.items():
                block, hashes = records_to_block(records, idxs, self.layer_name)
                yield step, block, hashes

    def __iter__(self):
        if self.device.type != "cuda":
            yield from self._host_blocks()
            return
        q: queue.Queue = queue.Queue(maxsize=self.prefetch)
        stop = threading.Event()
        reader = threading.Thread(target=self._host_files, args=(q, stop), daemon=True)
        reader.start()
        copy_stream = torch.cuda.Stream(self.device)
        self.h2d_bytes = 0

        def take():
            item = q.get()
            if isinstance(item, BaseException):
                raise item
            return item

        def upload(item):
            file_rel, by_step, payload, host = item
            with torch.cuda.stream(copy_stream):
                dev = host.to(self.device, non_blocking=True)
                done = torch.cuda.Event()
                done.record(copy_stream)
            self.h2d_bytes += host.numel()
            return file_rel, by_step, payload, dev, done

        try:
            nxt = take()
            pending = upload(nxt) if nxt is not None else None
            while pending is not None:
                nxt = take()
                ahead = upload(nxt) if nxt is not None else None  # the next file's copy overlaps this one's use
                file_rel, by_step, payload, dev, done = pending
                consumer = torch.cuda.current_stream(self.device)
                consumer.wait_event(done)
                dev.record_stream(consumer)
                records = self.store.records_from(payload, dev, file_rel)
                for step, idxs in by_step.items():
                    block, hashes = records_to_block(records, idxs, self.layer_name)
                    yield step, block, hashes
                pending = ahead
        finally:
            stop.set()
            reader.join(timeout=5)


class AsyncGradientWriter:
    """Background writer of record groups (async_writer.py:1-207): ``submit``
    records an event on the producer's stream, and one thread copies the group
    to the host on its own stream after that event, then writes it in
    submission order.  ``max_pending`` groups may wait; ``submit`` blocks beyond."""

    def __init__(self, store: GradientStore, *, max_pending: int = 2) -> None:
        self.store = store
        self._q: queue.Queue = queue.Queue(maxsize=max(1, int(max_pending)))
        self._error: BaseException | None = None
        self._streams: dict = {}
        self.locations: list[str] = []
        self._thread = threading.Thread(target=self._run, daemon=True)
        self._thread.start()
        self._closed = False

    def submit(self, records: list[GradientRecord]) -> None:
        if self._closed:
            raise RuntimeError("AsyncGradientWriter is closed")
        self._raise()
        events = {}
        for rec in records:
            dev = rec.gradient.device
            if dev.type == "cuda" and dev not in events:
                ev = torch.cuda.Event()
                ev.record(torch.cuda.current_stream(dev))
                events[dev] = ev
        self._q.put((records, events))

    def _run(self) -> None:
        while True:
            item = self._q.get()
            if item is None:
                self._q.task_done()
                return
            records, events = item
            try:
                host = []
                for rec in records:
                    dev = rec.gradient.device
                    if dev.type == "cuda":
                        stream = self._streams.setdefault(dev, torch.cuda.Stream(dev))
                        with torch.cuda.stream(stream):
                            stream.wait_event(events[dev])
                            g = _map_tensors(rec.gradient, lambda t: t.to("cpu"))
                    else:
                        g = rec.gradient
                    host.append(GradientRecord(rec.step, rec.input_hash, g, rec.sample_id_key))
                self.locations.append(self.store.save_bulk(host))
            except BaseException as exc:  # noqa: BLE001 - reported on the next call
                self._error = exc
            finally:
                self._q.task_done()

    def _raise(self) -> None:
        if self._error is not None:
            err, self._error = self._error, None
            raise err

    def flush(self) -> None:
        self._q.join()
        self._raise()

    def close(self) -> None:
        if not self._closed:
            self._closed = True
            self._q.put(None)
            self._thread.join()
            self._raise()

    def __enter__(self) -> AsyncGradientWriter:
        return self

    def __exit__(self, *_exc) -> bool:
        self.close()
        return False


__all__ = ["AsyncGradientWriter", "GradientStore", "PinnedBlockSource", "records_to_block"]

"""Device-direct loading of compressed-tensors (pack-quantized) checkpoints.

The reference loader (``quantization.py:325-430``) reads each safetensors shard
into host tensors, collects every expert of a layer, stacks them on the CPU
and copies the stacks into the module buffers; the model then moves to the
GPU.  Here a shard goes to the device whole:

* its header is parsed (the safetensors format: an 8-byte little-endian
  header length, a JSON header of ``{name: {dtype, shape, data_offsets}}``,
  then the tensor bytes), its data read by parallel positional reads into
  one reusable pinned host buffer and copied to the device in one transfer;
* each tensor is a view of that device copy, written straight into its
  destination: an expert's ``gate_proj`` / ``up_proj`` / ``down_proj``
  ``weight_packed`` / ``weight_scale`` into its slice of the stacked module
  buffers (gate rows before up rows, ``quantization.py:404-421``), every
  other tensor into the parameter or buffer of the same name.

No expert is staged on the host or stacked in a temporary: device memory
beyond the model is one shard.  The buffers keep the checkpoint layout (the
kernels read it directly), so no re-layout happens at load time.
"""
from __future__ import annotations

import json
import os
import struct
from pathlib import Path

import numpy as np
import torch

_DTYPES = {
    "BF16": torch.bfloat16, "F16": torch.float16, "F32": torch.float32, "F64": torch.float64,
    "I8": torch.int8, "U8": torch.uint8, "I16": torch.int16, "I32": torch.int32, "I64": torch.int64,
    "BOOL": torch.bool,
}

# expert tensor (projection, kind) -> tag
PROJ_TAGS = {
    ("gate_proj", "weight_packed"): "gp", ("gate_proj", "weight_scale"): "gs",
    ("up_proj", "weight_packed"): "up", ("up_proj", "weight_scale"): "us",
    ("down_proj", "weight_packed"): "dp", ("down_proj", "weight_scale"): "ds",
}


def parse_expert_key(key: str):
    """model.language_model.layers.{l}.experts.{e}.{proj}.{kind} -> (l, e, tag) or None."""
    if ".experts." not in key or not key.startswith("model.language_model.layers."):
        return None
    parts = key.split(".")
    if len(parts) != 8:
        return None
    tag = PROJ_TAGS.get((parts[6], parts[7]))
    if tag is None:
        return None
    return int(parts[3]), int(parts[5]), tag


def read_header(path: os.PathLike | str) -> tuple[dict, int]:
    """(tensor table, byte offset of the data section) of a safetensors file."""
    with open(path, "rb") as f:
        head = f.read(8)
        if len(head) != 8:
            raise ValueError(f"{path}: not a safetensors file")
        n = struct.unpack("<Q", head)[0]
        table = json.loads(f.read(n))
    table.pop("__metadata__", None)
    return table, 8 + n


def _view(raw: torch.Tensor, meta: dict) -> torch.Tensor:
    b, e = meta["data_offsets"]
    dt = _DTYPES[meta["dtype"]]
    t = raw[b:e]
    if b % torch.empty((), dtype=dt).element_size():
        t = t.clone()  # the view needs an element-aligned start
    return t.view(dt).view(meta["shape"])


def _pread_into(path, offset: int, buf: memoryview, threads: int) -> None:
    """Fill ``buf`` with the file's bytes from ``offset``, in ``threads`` parallel
    positional reads (each releases the GIL)."""
    from concurrent.futures import ThreadPoolExecutor

    size = len(buf)
    chunk = max(1 << 22, -(-size // max(1, threads)))
    fd = os.open(path, os.O_RDONLY)
    try:
        def read(lo: int) -> None:
            hi = min(size, lo + chunk)
            while lo < hi:
                n = os.preadv(fd, [buf[lo:hi]], offset + lo)
                if n <= 0:
                    raise ValueError(f"{path}: truncated data section")
                lo += n

        starts = list(range(0, size, chunk))
        if len(starts) == 1:
            read(0)
        else:
            with ThreadPoolExecutor(max_workers=len(starts)) as ex:
                list(ex.map(read, starts))
    finally:
        os.close(fd)


class ShardReader:
    """Whole-shard reads: host file -> pinned buffer -> one device copy."""

    def __init__(self, device, threads: int | None = None):
        self.device = torch.device(device)
        self._pinned: torch.Tensor | None = None
        self.bytes_read = 0
        self.threads = threads or min(16, len(os.sched_getaffinity(0)))

    def _staging(self, n: int) -> torch.Tensor:
        if self._pinned is None or self._pinned.numel() < n:
            self._pinned = torch.empty(n, dtype=torch.uint8, pin_memory=True)
        return self._pinned[:n]

    def open(self, path: os.PathLike | str) -> dict[str, torch.Tensor]:
        """Every tensor of the shard as a view of its data on this reader's device."""
        table, off = read_header(path)
        size = os.path.getsize(path) - off
        if self.device.type == "cpu":
            raw = torch.from_numpy(np.fromfile(path, dtype=np.uint8, offset=off, count=size))
        else:
            host = self._staging(size)
            _pread_into(path, off, memoryview(host.numpy()), self.threads)
            raw = host.to(self.device, non_blocking=False)
        self.bytes_read += size
        return {name: _view(raw, meta) for name, meta in table.items()}


class ExpertPlacer:
    """Writes per-expert checkpoint tensors into the stacked buffers of the
    4-bit experts modules (one per layer) and checks that every expert's six
    tensors arrived."""

    def __init__(self, modules: list):
        self.modules = modules
        self.seen = [set() for _ in modules]

    def place(self, layer: int, expert: int, tag: str, t: torch.Tensor) -> None:
        m = self.modules[layer]
        I = m.intermediate_dim
        if not 0 <= expert < m.num_experts:
            raise ValueError(f"layer {layer}: expert {expert} outside [0, {m.num_experts})")
        dst = {
            "gp": m.gate_up_packed[expert, :I], "up": m.gate_up_packed[expert, I:],
            "gs": m.gate_up_scale[expert, :I], "us": m.gate_up_scale[expert, I:],
            "dp": m.down_packed[expert], "ds": m.down_scale[expert],
        }[tag]
        if tuple(dst.shape) != tuple(t.shape):
            raise ValueError(f"layer {layer} expert {expert} {tag}: checkpoint shape {tuple(t.shape)} does not "
                             f"match the module's {tuple(dst.shape)} (group size {m.group_size})")
        dst.copy_(t)
        self.seen[layer].add((tag, expert))

    def check_complete(self) -> None:
        for layer, (m, seen) in enumerate(zip(self.modules, self.seen)):
            if seen and len(seen) != 6 * m.num_experts:
                raise ValueError(f"layer {layer}: {6 * m.num_experts - len(seen)} expert tensors missing from the "
                                 "checkpoint")


def shard_files(model_dir: Path) -> list[Path]:
    """The checkpoint's shard files (index order), or the single model.safetensors."""
    index_file = model_dir / "model.safetensors.index.json"
    if index_file.is_file():
        weight_map = json.loads(index_file.read_text(encoding="utf-8"))["weight_map"]
        return [model_dir / f for f in sorted(set(weight_map.values()))]
    return [model_dir / "model.safetensors"]


def stream_shards(files, placer: ExpertPlacer, targets: dict, device) -> int:
    """Load every shard onto ``device``: expert tensors through ``placer``, the rest
    into ``targets`` (name -> parameter / buffer).  Returns the bytes read."""
    reader = ShardReader(device)
    for path in files:
        tensors = reader.open(path)
        for key, val in tensors.items():
            if key.endswith(".weight_shape"):
                continue
            parsed = parse_expert_key(key)
            if parsed is not None:
                placer.place(*parsed, val)
            elif key in targets:
                tgt = targets[key]
                tgt.data.copy_(val.to(tgt.dtype) if val.is_floating_point() else val)
        del tensors
    placer.check_complete()
    return reader.bytes_read

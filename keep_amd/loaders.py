"""On-disk expert formats -> device tensors, and expert installs into slot rows.

Two formats hold the routed experts' E8P codes and row scales:

- ``layer-NN.npz`` (``scripts/runpod/v41_reap/keep_quant.py:125-133``): an
  uncompressed ``np.savez`` archive with ``{w1,w3,w2}_codes`` (uint16 E8P or
  uint8 E8, ``[E, N, K/8]``), ``{w1,w3,w2}_scales`` (fp16 ``[E, N, K/g]``) and
  ``code_bits`` (absent in the first E8P runs: 16, ``keep_quant.py:59-62``);
  w1 is gate, w3 up and w2 down (``omlx_lattice.py:583``). It is read by
  position, as ``Codes`` does (``scripts/v41_build/omlx_lattice.py:115-150``):
  every member must be stored uncompressed and in C order, and one expert's
  slab is a contiguous byte range of the file.
- safetensors ``{prefix}.codes`` / ``{prefix}.scales`` with an optional
  ``quantization_config`` metadata entry whose codebook SHA-256 must name one
  of the two E8 tables (``src/keep/io/load.py:102-114``); dimensions are
  inferred as ``infer_vq_linear_dims`` / ``infer_vq_switch_linear_dims`` do
  (``load.py:125-182``).

Reads go straight from the file into pinned host memory and from there to the
device with asynchronous copies; nothing is unpickled (``allow_pickle`` stays
off). ``ExpertInstaller`` is the install step of a residency runtime
(``omlx_routed.py:190-216``): it copies one expert's slabs into a slot of the
device pools on a side stream and hands back the copy's event, after which
the caller may route the expert (flip its router bias).
"""

from __future__ import annotations

import ctypes
import hashlib
import json
import os
import struct
import zipfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import numpy as np
import torch

from keep_amd import _lib

PROJECTIONS = (("gate", "w1"), ("up", "w3"), ("down", "w2"))


# --------------------------------------------------------------------------- codebook hashes


def _table_sha(name: str) -> str:
    buf = (ctypes.c_uint32 * 256)()
    _lib.check(getattr(_lib.load(), name)(buf), name)
    return hashlib.sha256(np.frombuffer(buf, dtype="<u4").tobytes()).hexdigest()


def codebook_sha256(code_bits: int) -> str:
    """SHA-256 of the packed table a code width indexes (``schema.py`` ``codebook_metadata_for_bits``)."""

    if code_bits == 16:
        return _table_sha("keep_e8p_packed_abs_grid")
    if code_bits == 8:
        return _table_sha("keep_e8_1bit_packed")
    raise ValueError("code_bits must be 8 or 16")


def validate_codebook_hash(metadata: dict) -> None:
    """``_validate_codebook_hash`` (``load.py:109-114``): a stated codebook hash must be one of ours."""

    raw = metadata.get("quantization_config")
    config = json.loads(raw) if raw is not None else {}
    codebook = config.get("codebook") if isinstance(config, dict) else None
    expected = codebook.get("sha256") if isinstance(codebook, dict) else None
    if expected is not None and expected not in {codebook_sha256(8), codebook_sha256(16)}:
        raise ValueError(f"checkpoint E8 codebook hash {expected!r} is not supported by this runtime")


# --------------------------------------------------------------------------- positional reads


def _pread_into(fd: int, offset: int, out: np.ndarray) -> int:
    view = memoryview(out.reshape(-1).view(np.uint8))
    done = 0
    while done < len(view):
        n = os.preadv(fd, [view[done:]], offset + done)
        if n <= 0:
            raise OSError(f"short read at offset {offset + done}")
        done += n
    return done


class _Members:
    """name -> (byte offset of the data, shape, dtype) of one file, with an open descriptor."""

    def __init__(self, path: Path, members: dict):
        self.path, self.members = path, members
        self.fd = os.open(path, os.O_RDONLY)

    def close(self) -> None:
        if getattr(self, "fd", -1) >= 0:  # a constructor that raised early opened nothing
            os.close(self.fd)
            self.fd = -1

    def __del__(self):
        self.close()

    def __contains__(self, name: str) -> bool:
        return name in self.members

    def info(self, name: str):
        if name not in self.members:
            raise KeyError(f"missing tensor {name!r} in {self.path}")
        return self.members[name]

    def slab(self, name: str, expert: int) -> tuple[int, int]:
        """(file offset, bytes) of ``name[expert]``."""

        start, shape, dtype = self.info(name)
        if not 0 <= expert < shape[0]:
            raise IndexError(f"expert {expert} out of range for {name} with {shape[0]} experts")
        size = int(np.prod(shape[1:], dtype=np.int64)) * dtype.itemsize
        return start + expert * size, size

    def read(self, name: str, experts=None, out: np.ndarray | None = None) -> np.ndarray:
        """``name[experts]`` read by position into ``out`` (allocated when None)."""

        _, shape, dtype = self.info(name)
        experts = range(shape[0]) if experts is None else list(experts)
        if out is None:
            out = np.empty((len(experts), *shape[1:]), dtype)
        if out.shape != (len(experts), *shape[1:]) or out.dtype != dtype or not out.flags.c_contiguous:
            raise ValueError(f"out must be a C-contiguous {dtype} array of shape {(len(experts), *shape[1:])}")
        for i, e in enumerate(experts):
            off, _ = self.slab(name, int(e))
            _pread_into(self.fd, off, out[i])
        return out


class LayerFile(_Members):
    """One ``layer-NN.npz`` of a keep_quant run, read by position."""

    def __init__(self, path):
        path = Path(path)
        members = {}
        with open(path, "rb") as raw, zipfile.ZipFile(path) as z:
            for info in z.infolist():
                if info.compress_type != zipfile.ZIP_STORED:
                    raise ValueError(f"{path}: {info.filename} is compressed; positional reads need np.savez")
                raw.seek(info.header_offset + 26)
                name_len, extra_len = struct.unpack("<HH", raw.read(4))
                with z.open(info) as f:
                    major, _ = np.lib.format.read_magic(f)
                    read = np.lib.format.read_array_header_1_0 if major == 1 else np.lib.format.read_array_header_2_0
                    shape, fortran, dtype = read(f)
                    if fortran:
                        raise ValueError(f"{path}: {info.filename} is stored in Fortran order")
                    if dtype.hasobject:
                        raise ValueError(f"{path}: {info.filename} holds Python objects")
                    start = info.header_offset + 30 + name_len + extra_len + f.tell()
                members[info.filename.removesuffix(".npy")] = (start, tuple(shape), dtype)
        super().__init__(path, members)
        if "code_bits" in members:
            self.code_bits = int(self.read_scalar("code_bits"))
        else:
            self.code_bits = 16  # the first E8P runs wrote no code_bits (keep_quant.py:62)
        if self.code_bits not in (8, 16):
            raise ValueError(f"{path}: code_bits must be 8 or 16, found {self.code_bits}")

    def read_scalar(self, name: str):
        start, shape, dtype = self.info(name)
        out = np.empty(shape, dtype)
        _pread_into(self.fd, start, out)
        return out.reshape(-1)[0] if out.size else None

    @property
    def num_experts(self) -> int:
        return self.info("w1_codes")[1][0]

    def dims(self, proj: str) -> tuple[int, int, int]:
        """(input_dims, output_dims, group_size) of projection ``w1`` / ``w3`` / ``w2``."""

        _, cshape, cdt = self.info(f"{proj}_codes")
        _, sshape, _ = self.info(f"{proj}_scales")
        want = np.uint16 if self.code_bits == 16 else np.uint8
        if len(cshape) != 3 or len(sshape) != 3 or cshape[:2] != sshape[:2]:
            raise ValueError(f"{proj}: codes {cshape} and scales {sshape} must be [E, N, *] alike")
        if cdt != want:
            raise ValueError(f"{proj}_codes must be {np.dtype(want)} for code_bits={self.code_bits}, found {cdt}")
        k = cshape[2] * 8
        if sshape[2] <= 0 or k % sshape[2]:
            raise ValueError(f"{proj}: scale count must divide the inferred input dims")
        return k, cshape[1], k // sshape[2]


class SafetensorsFile(_Members):
    """A safetensors file read by position; ``metadata`` is its ``__metadata__``."""

    _DT = {"U8": np.uint8, "UINT8": np.uint8, "U16": np.uint16, "UINT16": np.uint16, "F16": np.float16,
           "F32": np.float32, "BF16": np.uint16, "I16": np.int16, "I32": np.int32, "U32": np.uint32}

    def __init__(self, path):
        path = Path(path)
        with open(path, "rb") as f:
            (n,) = struct.unpack("<Q", f.read(8))
            header = json.loads(f.read(n))
        self.metadata = header.pop("__metadata__", {}) or {}
        self.dtypes = {}
        members = {}
        for name, t in header.items():
            dt = t["dtype"].upper()
            if dt not in self._DT:
                raise ValueError(f"{path}: {name} has unsupported dtype {t['dtype']}")
            begin, end = t["data_offsets"]
            shape = tuple(t["shape"])
            np_dt = np.dtype(self._DT[dt])
            if end - begin != int(np.prod(shape, dtype=np.int64)) * np_dt.itemsize:
                raise ValueError(f"{path}: {name} byte range does not match its shape")
            members[name] = (8 + n + begin, shape, np_dt)
            self.dtypes[name] = dt
        super().__init__(path, members)

    def _code_bits(self, name: str) -> int:
        dt = self.dtypes[name]
        if dt in ("U8", "UINT8"):
            return 8
        if dt in ("U16", "UINT16"):
            return 16
        raise ValueError(f"{name} must be uint8 or uint16, found {dt}")

    def infer_vq_linear_dims(self, prefix: str) -> tuple[int, int, int, int]:
        """(in_dim, out_dim, group_size, code_bits) of a 2-D projection (``load.py:125-151``)."""

        codes, scales = self.info(f"{prefix}.codes")[1], self.info(f"{prefix}.scales")[1]
        if len(codes) != 2:
            raise ValueError(f"{prefix}.codes must be 2D, found {codes}")
        if len(scales) != 2:
            raise ValueError(f"{prefix}.scales must be 2D, found {scales}")
        if codes[0] != scales[0]:
            raise ValueError("codes and scales must have the same out_dim")
        bits = self._code_bits(f"{prefix}.codes")
        in_dim = codes[1] * 8
        if scales[1] <= 0 or in_dim % scales[1]:
            raise ValueError("scale count must divide inferred in_dim")
        return in_dim, codes[0], in_dim // scales[1], bits

    def infer_vq_switch_linear_dims(self, prefix: str) -> tuple[int, int, int, int, int]:
        """(in_dim, out_dim, num_experts, group_size, code_bits) (``load.py:154-182``)."""

        codes, scales = self.info(f"{prefix}.codes")[1], self.info(f"{prefix}.scales")[1]
        if len(codes) != 3:
            raise ValueError(f"{prefix}.codes must be 3D [experts, out, in/8], found {codes}")
        if len(scales) != 3:
            raise ValueError(f"{prefix}.scales must be 3D [experts, out, in/group], found {scales}")
        if codes[:2] != scales[:2]:
            raise ValueError("switch codes and scales must have the same expert and out dimensions")
        bits = self._code_bits(f"{prefix}.codes")
        in_dim = codes[2] * 8
        if scales[2] <= 0 or in_dim % scales[2]:
            raise ValueError("switch scale count must divide inferred in_dim")
        return in_dim, codes[1], codes[0], in_dim // scales[2], bits


# --------------------------------------------------------------------------- device loads


def _to_device(src: _Members, name: str, experts, device) -> torch.Tensor:
    """``name[experts]`` -> a device tensor through one pinned staging buffer and an async copy."""

    _, shape, dtype = src.info(name)
    n = shape[0] if experts is None else len(list(experts))
    tdt = {1: torch.uint8, 2: torch.int16, 4: torch.int32}[dtype.itemsize] if dtype.kind in "ui" else \
        {np.dtype(np.float16): torch.float16, np.dtype(np.float32): torch.float32}[dtype]
    host = torch.empty((n, *shape[1:]), dtype=tdt, pin_memory=True)
    src.read(name, experts, host.numpy().view(dtype))
    dev = torch.empty(host.shape, dtype=tdt, device=device)
    dev.copy_(host, non_blocking=True)
    if getattr(src, "dtypes", {}).get(name) == "BF16":
        dev = dev.view(torch.bfloat16)
    return dev


def load_switch_glu_npz(path, *, device, experts=None):
    """``QuantizedVQSwitchGLU`` (gate = w1, up = w3, down = w2) from a ``layer-NN.npz``.

    ``experts`` selects and orders the experts held (slot s = ``experts[s]``); all by default."""

    from keep_amd.nn import QuantizedVQSwitchGLU, QuantizedVQSwitchLinear

    lf = LayerFile(path)
    device = torch.device(device)
    exp = None if experts is None else [int(e) for e in experts]
    mods = {}
    for role, proj in PROJECTIONS:
        k, n, g = lf.dims(proj)
        codes = _to_device(lf, f"{proj}_codes", exp, device)
        scales = _to_device(lf, f"{proj}_scales", exp, device)
        mods[role] = QuantizedVQSwitchLinear(input_dims=k, output_dims=n, num_experts=codes.shape[0], codes=codes,
                                             scales=scales, group_size=g, code_bits=lf.code_bits)
    torch.cuda.current_stream(device).synchronize()  # the pinned staging buffers are released here
    lf.close()
    return QuantizedVQSwitchGLU(gate_proj=mods["gate"], up_proj=mods["up"], down_proj=mods["down"])


def load_switch_linear_safetensors(path, prefix: str, *, device):
    """``QuantizedVQSwitchLinear`` from ``{prefix}.codes`` / ``{prefix}.scales`` of a safetensors file
    (codebook hash checked, dimensions inferred)."""

    from keep_amd.nn import QuantizedVQSwitchLinear

    st = SafetensorsFile(path)
    validate_codebook_hash(st.metadata)
    k, n, e, g, bits = st.infer_vq_switch_linear_dims(prefix)
    device = torch.device(device)
    codes = _to_device(st, f"{prefix}.codes", None, device)
    scales = _to_device(st, f"{prefix}.scales", None, device)
    torch.cuda.current_stream(device).synchronize()
    st.close()
    return QuantizedVQSwitchLinear(input_dims=k, output_dims=n, num_experts=e, codes=codes, scales=scales,
                                   group_size=g, code_bits=bits)


# torch dtypes that hold a file array's bits unchanged (codes are copied as
# raw bits; the scales keep their floating-point type)
_POOL_DTYPES = {"u2": (torch.int16, torch.uint16), "i2": (torch.int16, torch.uint16),
                "u1": (torch.uint8, torch.int8), "i1": (torch.uint8, torch.int8),
                "f2": (torch.float16,), "f4": (torch.float32,)}


class ExpertInstaller:
    """Installs experts from a ``LayerFile`` into slot rows of device pools.

    ``pools`` maps a projection (``w1`` / ``w3`` / ``w2``) to its device
    ``(codes [S, N, K/8], scales [S, N, K/g])`` slot arrays. ``submit`` reads
    the expert's six slabs into pinned memory and queues their copies on the
    installer's own stream (default priority), after the work already queued
    on the caller's current stream; it returns the event that completes with
    the copies. Pool dtypes must hold the file's bits unchanged (uint16 /
    int16 codes for uint16 files, float16 scales for float16 ones). Only once ``ready(event)`` holds may the caller
    route the expert (clear its router bias), and a slot may only be
    overwritten once no call that can still route to it is in flight, as the
    reference's cooling rule requires (``omlx_routed.py:218-236``).
    """

    def __init__(self, layer: LayerFile, pools: dict, device):
        self.layer, self.pools = layer, pools
        self.device = torch.device(device)
        self.stream = torch.cuda.Stream(device=self.device)
        self._pool = ThreadPoolExecutor(max_workers=8, thread_name_prefix="keep-install")
        self._held: list[tuple[torch.cuda.Event, list]] = []
        for proj, (codes, scales) in pools.items():
            for name, dst in ((f"{proj}_codes", codes), (f"{proj}_scales", scales)):
                _, shape, dtype = layer.info(name)
                if tuple(dst.shape[1:]) != tuple(shape[1:]):
                    raise ValueError(f"pool for {name} must be [S, {', '.join(map(str, shape[1:]))}], "
                                     f"found {tuple(dst.shape)}")
                ok = _POOL_DTYPES.get(np.dtype(dtype).str.lstrip("<>|="), ())
                if dst.dtype not in ok:
                    raise ValueError(f"pool for {name} must hold the file's {np.dtype(dtype).name} bits "
                                     f"({' or '.join(str(d) for d in ok) or 'no torch dtype'}), found {dst.dtype}")

    CHUNK = 1 << 20  # bytes per positional read; the pieces of one expert are read in parallel

    def submit(self, expert: int, slot: int) -> torch.cuda.Event:
        staged, reads = [], []
        for proj, (codes, scales) in self.pools.items():
            for name, dst in ((f"{proj}_codes", codes), (f"{proj}_scales", scales)):
                if not 0 <= slot < dst.shape[0]:
                    raise IndexError(f"slot {slot} out of range for a pool of {dst.shape[0]}")
                off, size = self.layer.slab(name, int(expert))
                host = torch.empty(dst.shape[1:], dtype=dst.dtype, pin_memory=True)
                raw = host.numpy().reshape(-1).view(np.uint8)
                for c in range(0, size, self.CHUNK):
                    reads.append(self._pool.submit(_pread_into, self.layer.fd, off + c, raw[c:c + self.CHUNK]))
                staged.append((dst, host))
        for r in reads:
            r.result()
        # pool writes already queued on the caller's stream land before the install copies
        self.stream.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(self.stream):
            for dst, host in staged:
                dst[slot].copy_(host, non_blocking=True)
            ev = torch.cuda.Event()
            ev.record(self.stream)
        staged = [host for _, host in staged]
        self._held.append((ev, staged))
        return ev

    def ready(self, event: torch.cuda.Event) -> bool:
        done = event.query()
        self._held = [(e, s) for e, s in self._held if not e.query()]
        return done

"""Reading .vn model files straight onto the GPU.

A .vn file (packages/verse_torch/verse_torch/vn_format.py:1-60, format version
VN_FORMAT_VERSION = 2, :99) is a ZIP container holding meta.json, config.yml
and the weights as model.safetensors, or model.npz where safetensors was not
installed (a stored ZIP of .npy entries, :231-244).  The writer deflates every
entry (:312-313), so the weights cannot be memory-mapped from the container;
the reference extracts them to a temporary file and maps that
(VNFileReader.read_weights, :598-650).

VNReader keeps VNFileReader's checks (meta.json required, format version 1 or
2, config.yml required, safetensors preferred over npz; :543-620) and streams
the weights instead: the weights entry is inflated once, front to back, and
each tensor is handed out in row chunks, so host memory holds one chunk at a
time.  load_vn_weights copies every chunk to the device and, for the matrices
the draft runs as INT4 group-128 GEMVs, quantizes it there (vnx_quantize_w4_g)
into the final packed buffers: no full-precision copy of a quantized matrix
exists on the host or the device.  The tied embedding becomes both the INT4
LM head and the bf16 lookup table in the same pass.
"""
from __future__ import annotations

import ast
import ctypes
import json
import struct
import zipfile
from typing import Callable, Dict, Iterator, Optional, Tuple

import numpy as np
import torch

from . import _lib

META_NAME = "meta.json"
CONFIG_NAME = "config.yml"
WEIGHTS_ST = "model.safetensors"
WEIGHTS_NPZ = "model.npz"

# safetensors dtype tags -> (torch dtype, bytes per element)
_ST_DTYPES = {
    "F64": (torch.float64, 8), "F32": (torch.float32, 4), "F16": (torch.float16, 2), "BF16": (torch.bfloat16, 2),
    "I64": (torch.int64, 8), "I32": (torch.int32, 4), "I16": (torch.int16, 2), "I8": (torch.int8, 1),
    "U8": (torch.uint8, 1), "BOOL": (torch.bool, 1),
}
_NP_DTYPES = {
    "<f8": "F64", "<f4": "F32", "<f2": "F16", "<i8": "I64", "<i4": "I32", "<i2": "I16", "|i1": "I8", "|u1": "U8",
    "|b1": "BOOL",
}
_VNX_DTYPE = {"F32": _lib.VNX_F32, "BF16": _lib.VNX_BF16, "F16": _lib.VNX_F16}


def _read_exact(f, n: int, into: Optional[memoryview] = None) -> memoryview:
    """n bytes from the stream f (into `into` when given)."""
    buf = into if into is not None else memoryview(bytearray(n))
    got = 0
    while got < n:
        r = f.readinto(buf[got:n])
        if not r:
            raise ValueError(".vn weights entry ended early")
        got += r
    return buf[:n]


class TensorStream:
    """One tensor of the weights entry: name, dtype tag, shape, and its bytes
    read front to back with read_into(buf, nrows) (rows along the first axis)."""

    def __init__(self, f, name: str, dtype: str, shape: Tuple[int, ...]):
        self._f = f
        self.name = name
        self.dtype = dtype
        self.shape = tuple(int(s) for s in shape)
        self.itemsize = _ST_DTYPES[dtype][1]
        self.rows = self.shape[0] if self.shape else 1
        self.row_bytes = self.itemsize * int(np.prod(self.shape[1:], dtype=np.int64)) if self.shape else self.itemsize
        self.nbytes = self.rows * self.row_bytes
        self._left = self.nbytes

    def read_into(self, buf: memoryview, nrows: int) -> memoryview:
        n = nrows * self.row_bytes
        if n > self._left:
            raise ValueError(f"{self.name}: reading past the tensor")
        self._left -= n
        return _read_exact(self._f, n, buf)

    def skip_rest(self) -> None:
        while self._left:
            n = min(self._left, 1 << 24)
            _read_exact(self._f, n)
            self._left -= n


class VNReader:
    """A .vn file's meta, config and streamed weights (VNFileReader,
    vn_format.py:527-650, with streaming in place of the temporary file)."""

    def __init__(self, path: str):
        self.path = str(path)
        self._zf = zipfile.ZipFile(self.path, "r")
        self._names = set(self._zf.namelist())
        self._meta = None
        self.vn_format_version = 1

    def close(self) -> None:
        self._zf.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def read_meta(self) -> dict:
        """meta.json; format version 1 (no field) or 2, else ValueError."""
        if self._meta is not None:
            return self._meta
        if META_NAME not in self._names:
            raise ValueError(f".vn file has no {META_NAME}: {self.path}")
        meta = json.loads(self._zf.read(META_NAME).decode("utf-8"))
        version = meta.get("vn_format_version", 1)
        if version not in (1, 2):
            raise ValueError(f"unsupported .vn format version: expected 1 or 2, got {version}")
        self.vn_format_version = version
        self._meta = meta
        return meta

    @property
    def weight_format(self) -> str:
        return self.read_meta().get("weight_format", "npz")

    def read_config(self) -> dict:
        """config.yml as a dict (YAML via safe_load, or its JSON subset)."""
        if CONFIG_NAME not in self._names:
            raise ValueError(f".vn file has no {CONFIG_NAME}: {self.path}")
        text = self._zf.read(CONFIG_NAME).decode("utf-8")
        try:
            import yaml
            loaded = yaml.safe_load(text)
        except ImportError:
            loaded = json.loads(text)
        return loaded if isinstance(loaded, dict) else {}

    def tensors(self) -> Iterator[TensorStream]:
        """Every weight tensor in file order, streamed from the inflating
        entry; a tensor the caller does not read to the end is skipped."""
        self.read_meta()
        if WEIGHTS_ST in self._names and self.weight_format == "safetensors":
            yield from self._safetensors()
        elif WEIGHTS_NPZ in self._names:
            yield from self._npz()
        elif WEIGHTS_ST in self._names:
            yield from self._safetensors()
        else:
            raise ValueError(f".vn file has no weights entry: {self.path}")

    def _safetensors(self) -> Iterator[TensorStream]:
        # 8-byte little-endian header length, a JSON header {name: {dtype,
        # shape, data_offsets: [begin, end)}}, then the data section
        with self._zf.open(WEIGHTS_ST) as f:
            (hlen,) = struct.unpack("<Q", bytes(_read_exact(f, 8)))
            if hlen > 1 << 28:
                raise ValueError("safetensors header too large")
            header = json.loads(bytes(_read_exact(f, hlen)).decode("utf-8"))
            header.pop("__metadata__", None)
            entries = sorted(header.items(), key=lambda kv: kv[1]["data_offsets"][0])
            pos = 0
            for name, e in entries:
                b, end = (int(x) for x in e["data_offsets"])
                if b < pos:
                    raise ValueError("overlapping safetensors entries")
                if b > pos:
                    _read_exact(f, b - pos)
                if e["dtype"] not in _ST_DTYPES:
                    raise ValueError(f"{name}: unsupported dtype {e['dtype']}")
                t = TensorStream(f, name, e["dtype"], e["shape"])
                if t.nbytes != end - b:
                    raise ValueError(f"{name}: {end - b} bytes for shape {t.shape}")
                yield t
                t.skip_rest()
                pos = end

    def _npz(self) -> Iterator[TensorStream]:
        # a stored (uncompressed) ZIP of NAME.npy entries, read through its
        # local file headers; each .npy: magic, version, header dict, data
        with self._zf.open(WEIGHTS_NPZ) as f:
            while True:
                sig = bytes(f.read(4))
                if sig != b"PK\x03\x04":
                    return  # central directory (or the end): no more entries
                hdr = bytes(_read_exact(f, 26))
                _, flags, method, _, _, _, csize, usize, nlen, xlen = struct.unpack("<HHHHHIIIHH", hdr)
                name = bytes(_read_exact(f, nlen)).decode("utf-8")
                extra = bytes(_read_exact(f, xlen))
                if method != 0:
                    raise ValueError(f"npz entry {name} is compressed")
                if flags & 0x08:
                    raise ValueError(f"npz entry {name} has no sizes in its header")
                if usize == 0xFFFFFFFF:  # ZIP64: sizes in the extra field (tag 1)
                    i = 0
                    while i + 4 <= len(extra):
                        tag, sz = struct.unpack("<HH", extra[i:i + 4])
                        if tag == 1:
                            usize = struct.unpack("<Q", extra[i + 4:i + 12])[0]
                            break
                        i += 4 + sz
                magic = bytes(_read_exact(f, 8))
                if magic[:6] != b"\x93NUMPY":
                    raise ValueError(f"npz entry {name} is not a .npy")
                major = magic[6]
                hl = struct.unpack("<H" if major == 1 else "<I", bytes(_read_exact(f, 2 if major == 1 else 4)))[0]
                d = ast.literal_eval(bytes(_read_exact(f, hl)).decode("latin1"))
                if d.get("fortran_order"):
                    raise ValueError(f"npz entry {name} is Fortran-ordered")
                tag = _NP_DTYPES.get(d["descr"])
                if tag is None:
                    raise ValueError(f"npz entry {name}: unsupported dtype {d['descr']}")
                key = name[:-4] if name.endswith(".npy") else name
                t = TensorStream(f, key, tag, d["shape"])
                data_bytes = usize - (8 + (2 if major == 1 else 4) + hl)
                if t.nbytes != data_bytes:
                    raise ValueError(f"npz entry {name}: {data_bytes} bytes for shape {t.shape}")
                yield t
                t.skip_rest()


class Int4Weight:
    """An INT4 group-128 weight already on the device: packed (N, K/2) uint8
    and fp16 scales (N, K/128); `dense`, when set, is a copy in the compute
    dtype (the tied embedding's lookup table)."""

    def __init__(self, wq: torch.Tensor, sc: torch.Tensor, dense: Optional[torch.Tensor] = None):
        self.wq, self.sc, self.dense = wq, sc, dense
        self.shape = (wq.shape[0], wq.shape[1] * 2)

    @staticmethod
    def cat(ws) -> "Int4Weight":
        return Int4Weight(torch.cat([w.wq for w in ws], 0), torch.cat([w.sc for w in ws], 0))


def int4_matrix(name: str, shape) -> bool:
    """The matrices a draft runs as INT4 GEMVs: attention projections, the
    SwiGLU FFN of 'trisparse' layers, the embedding and an untied LM head
    (MoD experts stay dense), K a multiple of 128."""
    if len(shape) != 2 or shape[1] % 128:
        return False
    if name in ("tok_emb.weight", "head.weight"):
        return True
    if ".parts." in name or ".router" in name:
        return False
    return any(name.endswith(s) for s in ("attn.wq.weight", "attn.wk.weight", "attn.wv.weight", "attn.proj.weight",
                                          "ffn.w_gate.weight", "ffn.w_up.weight", "ffn.w_down.weight"))


def load_vn_weights(reader: VNReader, hip, quantize: Callable[[str, tuple], bool] = int4_matrix,
                    dense_dtype=torch.bfloat16, chunk_bytes: int = 64 << 20,
                    skip: Callable[[str], bool] = lambda name: False) -> Dict[str, object]:
    """{name: Int4Weight or device tensor} from the streamed weights.

    Matrices `quantize` selects go through vnx_quantize_w4_g chunk by chunk
    (the embedding also keeps a dense_dtype copy for lookups); every other
    tensor is copied to the device as stored (float64 as float32); names
    `skip` selects are read past without a copy.  Two
    pinned host buffers and two device buffers of chunk_bytes alternate, so
    inflating a chunk overlaps the copy and quantization of the previous."""
    dev = hip.torch_device
    stream = torch.cuda.current_stream(dev)
    L = hip._L
    host = [torch.empty(chunk_bytes, dtype=torch.uint8, pin_memory=True) for _ in range(2)]
    stage = [torch.empty(chunk_bytes, dtype=torch.uint8, device=dev) for _ in range(2)]
    done = [torch.cuda.Event(), torch.cuda.Event()]
    for e in done:
        e.record(stream)
    bad = torch.zeros(1, dtype=torch.int32, device=dev)
    out: Dict[str, object] = {}
    slot = 0
    for t in reader.tensors():
        if skip(t.name):
            continue
        if t.row_bytes > chunk_bytes:
            raise ValueError(f"{t.name}: a row of {t.row_bytes} bytes exceeds the {chunk_bytes}-byte chunk")
        tdt = _ST_DTYPES[t.dtype][0]
        q = quantize(t.name, t.shape) and t.dtype in _VNX_DTYPE
        if q:
            N, K = t.shape
            wq = torch.empty((N, K // 2), dtype=torch.uint8, device=dev)
            sc = torch.empty((N, K // 128), dtype=torch.float16, device=dev)
            dense = torch.empty((N, K), dtype=dense_dtype, device=dev) if t.name == "tok_emb.weight" else None
        else:
            dst = torch.empty(t.shape, dtype=torch.float32 if tdt == torch.float64 else tdt, device=dev)
            flat = dst.view(t.rows, -1) if t.shape else dst.view(1, 1)
        per = max(1, chunk_bytes // t.row_bytes)
        r0 = 0
        while r0 < t.rows:
            n = min(per, t.rows - r0)
            done[slot].synchronize()          # this slot's previous copy and kernel are finished
            h = host[slot]
            t.read_into(memoryview(h.numpy()), n)
            nb = n * t.row_bytes
            d = stage[slot][:nb]
            d.copy_(h[:nb], non_blocking=True)
            src = d.view(tdt).view(n, -1)
            if q:
                _lib.check(L.vnx_quantize_w4_g(
                    ctypes.c_void_p(src.data_ptr()), _VNX_DTYPE[t.dtype], n, K, K, 128,
                    ctypes.c_void_p(wq[r0].data_ptr()), wq.stride(0), ctypes.c_void_p(sc[r0].data_ptr()), sc.stride(0),
                    ctypes.c_void_p(bad.data_ptr()), ctypes.c_void_p(stream.cuda_stream)), "quantize_w4_g")
                if dense is not None:
                    dense[r0:r0 + n].copy_(src)
            else:
                flat[r0:r0 + n].copy_(src)
            done[slot].record(stream)
            slot ^= 1
            r0 += n
        out[t.name] = Int4Weight(wq, sc, dense) if q else dst
    torch.cuda.synchronize(dev)
    if int(bad.item()):
        raise ValueError(f"{int(bad.item())} weight groups hold non-finite values or a scale that underflows fp16")
    return out


def config_from_vn(conf: dict, weights: Dict[str, object], name: str = ""):
    """ModelConfig from a .vn config.yml: CometSparkNexLM.get_config
    (cometspark.py:1207-1256: dim, no embedding scale) or CometSparkV05Config
    (spark/src/base_config.py:182-260: n_embd, embedding_scale, layer_pattern
    None -> 'mod' every mod_every layers; temperature_scaling :266).  Both
    carry tie_weights (cometspark.py:1233, base_config.py:239).  The SwiGLU
    hidden size comes from the stored w_gate rows when they differ from the
    default."""
    from .model import ModelConfig, v02_pattern
    v05 = "n_embd" in conf
    dim = int(conf["n_embd"] if v05 else conf["dim"])
    n_layer = int(conf["n_layer"])
    pattern = conf.get("layer_pattern")
    if pattern is None:
        if conf.get("use_vda"):
            raise ValueError("layer_pattern None with use_vda is not supported")
        pattern = v02_pattern(n_layer, int(conf.get("mod_every", 4)))
    n_head = int(conf["n_head"])
    mlp_hidden = None
    for i, kind in enumerate(pattern):
        w = weights.get(f"blocks.{i}.ffn.w_gate.weight")
        if kind == "trisparse" and w is not None:
            mlp_hidden = int(w.shape[0])
            break
    return ModelConfig(
        vocab_size=int(conf["vocab_size"]), dim=dim, n_layer=n_layer, n_head=n_head,
        n_kv_head=int(conf.get("n_kv_head") or n_head), layer_pattern=list(pattern),
        window_size=int(conf.get("window_size", 1024)), num_global_tokens=int(conf.get("num_global_tokens", 128)),
        use_alibi=bool(conf.get("use_alibi", False)), use_rope=bool(conf.get("use_rope", True)),
        rope_theta=float(conf.get("rope_theta", 10000.0)), num_dense_parts=int(conf.get("num_dense_parts", 4)),
        num_experts_per_part=int(conf.get("num_experts_per_part", 4)), top_k=int(conf.get("top_k", 2)),
        expert_hidden=conf.get("expert_hidden"), mlp_hidden=mlp_hidden,
        embedding_scale=bool(conf.get("embedding_scale", True)) if v05 else False,
        tie_weights=bool(conf.get("tie_weights", True)),
        temperature_scaling=float(conf.get("temperature_scaling", 1.0)) if v05 else 1.0, name=name)


__all__ = ["VNReader", "TensorStream", "Int4Weight", "int4_matrix", "load_vn_weights", "config_from_vn"]

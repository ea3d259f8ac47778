"""Writes .vn files in the layout of the reference's VNFileWriter
(packages/verse_torch/verse_torch/vn_format.py:266-382, :479-500): a
ZIP_DEFLATED container with meta.json (vn_format_version 2, arch, weight
format, weight count), config.yml (yaml.safe_dump) and model.safetensors, or
model.npz as a stored ZIP of NAME.npy entries (:231-244).  Test data only."""
import io
import json
import os
import tempfile
import zipfile

import numpy as np
import yaml


def write_vn(path, state, config, fmt="safetensors", version=2, bf16_names=(), drop=()):
    """state {name: float32 ndarray}; names in bf16_names are stored as BF16
    (safetensors only); entries named in drop are left out of the container."""
    meta = {"arch": "versenex", "weight_format": fmt, "compression_info": None,
            "created_at": "2026-01-01T00:00:00", "weight_count": len(state), "has_training_state": False,
            "has_optimizer_state": False, "has_extra_state": False}
    if version is not None:
        meta["vn_format_version"] = version
    with zipfile.ZipFile(path, "w", zipfile.ZIP_DEFLATED) as zf:
        if fmt == "safetensors":
            if bf16_names:
                import torch
                from safetensors.torch import save_file
                tens = {k: (torch.from_numpy(np.ascontiguousarray(v)).to(torch.bfloat16) if k in bf16_names
                            else torch.from_numpy(np.ascontiguousarray(v))) for k, v in state.items()}
            else:
                from safetensors.numpy import save_file
                tens = {k: np.ascontiguousarray(v) for k, v in state.items()}
            fd, tmp = tempfile.mkstemp(suffix=".safetensors")
            os.close(fd)
            try:
                save_file(tens, tmp)
                with open(tmp, "rb") as f:
                    payload = f.read()
            finally:
                os.remove(tmp)
            if "weights" not in drop:
                zf.writestr("model.safetensors", payload)
        else:
            buf = io.BytesIO()
            with zipfile.ZipFile(buf, "w", zipfile.ZIP_STORED) as inner:
                for k, v in state.items():
                    nb = io.BytesIO()
                    np.lib.format.write_array(nb, np.ascontiguousarray(v), allow_pickle=False)
                    inner.writestr(f"{k}.npy", nb.getvalue())
            if "weights" not in drop:
                zf.writestr("model.npz", buf.getvalue())
        if "config" not in drop:
            zf.writestr("config.yml", yaml.safe_dump(config, sort_keys=False))
        if "meta" not in drop:
            zf.writestr("meta.json", json.dumps(meta))

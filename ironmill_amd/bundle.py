"""`.ironml-gpu` bundle reader (and a writer of the same layout) for the HIP backend.

A bundle is a directory holding ``manifest.json`` and the weight files under
``weights/`` (ironmill-compile/src/gpu/bundle.rs:1-19):

* ``format_version`` 1, ``model_config`` (architecture, sizes, rms_norm_eps,
  rope_theta, ...), ``quantization`` and ``tensors``
  (ironmill-core/src/gpu/bundle.rs:34-150);
* a tensor is ``{"format": "dense", "file", "shape", "dtype"}`` or
  ``{"format": "affine_dequantize", "quantized_data_file", "scales_file",
  "zeros_file", "shape", "bit_width", "group_size", "axis", "dtype",
  "awq_scales_file"?, "g_idx_file"?, "scale_dtype"?, "zero_point_dtype"?}``;
  scales and zero-points are stored in their original dtype (f32 from the
  quantizer), AWQ scales as f16 (quantized.rs:994-1007).

``GpuBundle`` is the counterpart of ``MetalBundleProvider``
(ironmill-inference/src/metal/bundle.rs:18-91) over
``read_tensor_from_manifest`` (ironmill-core/src/gpu/bundle.rs:300-420); the
device upload of an affine tensor converts scales and zero-points to f16 with
round-to-nearest-even, as ``load_weight_buffer`` does (metal/weights.rs:
1036-1114, core/dequant.rs:305-345), and keeps the codes as stored.
``load_decoder`` walks the standard transformer layout of
``load_model_weights`` (ironmill-inference/src/weight_loading.rs:162-300).
"""
from __future__ import annotations

import json
import os

import numpy as np

from . import ops, quant

FORMAT_VERSION = 1

# scalar type names of the manifest (ironmill-core/src/gpu/bundle.rs:150-200)
_DTYPES = {
    "float16": np.float16, "float32": np.float32, "float64": np.float64, "int8": np.int8,
    "int16": np.int16, "int32": np.int32, "int64": np.int64, "uint8": np.uint8, "uint16": np.uint16,
    "uint32": np.uint32, "uint64": np.uint64, "bool": np.bool_,
}
_REQUIRED_CONFIG = ("architecture", "hidden_size", "intermediate_size", "num_hidden_layers",
                    "num_attention_heads", "num_key_value_heads", "head_dim", "vocab_size",
                    "max_position_embeddings", "rms_norm_eps", "rope_theta")


class BundleError(ValueError):
    """A malformed bundle or a missing tensor (MetalError::WeightLoading / MilError)."""


def sanitize(name: str) -> str:
    """Tensor name -> file name component (dots and slashes to underscores, bundle.rs:38-43)."""
    return name.replace(".", "_").replace("/", "_")


def _dtype(name: str):
    try:
        return _DTYPES[name]
    except KeyError:
        raise BundleError(f"unknown scalar type: {name}") from None


def to_f16_params(raw: np.ndarray) -> np.ndarray:
    """convert_params_to_f16 (core/dequant.rs:305-345): f16 as is, anything else through f32
    rounded to nearest even."""
    if raw.dtype == np.float16:
        return raw.copy()
    return raw.astype(np.float32).astype(np.float16)


class GpuBundle:
    """A `.ironml-gpu` directory opened for reading (MetalBundleProvider)."""

    def __init__(self, path: str):
        self.path = os.fspath(path)
        mpath = os.path.join(self.path, "manifest.json")
        try:
            with open(mpath) as f:
                text = f.read()
        except OSError as e:
            raise BundleError(f"failed to read manifest at {mpath}: {e}") from None
        try:
            self.manifest = json.loads(text)
        except json.JSONDecodeError as e:
            raise BundleError(f"failed to parse manifest: {e}") from None
        version = self.manifest.get("format_version")
        if version != FORMAT_VERSION:
            raise BundleError(f"unsupported bundle format version: {version}")
        cfg = self.manifest.get("model_config")
        if not isinstance(cfg, dict):
            raise BundleError("model_config must be an object")
        for key in _REQUIRED_CONFIG:
            if key not in cfg:
                raise BundleError(f"missing field in model_config: {key}")
        self.config = dict(cfg)
        self.config.setdefault("tie_word_embeddings", False)
        self.tensors = self.manifest.get("tensors") or {}

    def tensor_names(self):
        return list(self.tensors)

    def has_tensor(self, name: str) -> bool:
        return name in self.tensors

    def _desc(self, name: str) -> dict:
        desc = self.tensors.get(name)
        if desc is None:
            raise BundleError(f"tensor not found in bundle: {name}")
        return desc

    def _read(self, rel: str, dtype) -> np.ndarray:
        try:
            with open(os.path.join(self.path, rel), "rb") as f:
                return np.frombuffer(f.read(), dtype=dtype)
        except OSError as e:
            raise BundleError(f"failed to read {rel}: {e}") from None

    def tensor(self, name: str) -> dict:
        """The stored tensor as host arrays (read_tensor_from_manifest)."""
        d = self._desc(name)
        fmt = d.get("format")
        if fmt == "dense":
            arr = self._read(d["file"], _dtype(d["dtype"]))
            return {"format": fmt, "data": arr.reshape(d["shape"]), "shape": list(d["shape"])}
        if fmt == "affine_dequantize":
            # scale / zero dtypes default to float16 when the manifest omits them
            sdt = _dtype(d.get("scale_dtype") or "float16")
            zdt = _dtype(d.get("zero_point_dtype") or "float16")
            out = {"format": fmt, "data": self._read(d["quantized_data_file"], np.uint8),
                   "scales": self._read(d["scales_file"], sdt), "zeros": self._read(d["zeros_file"], zdt),
                   "shape": list(d["shape"]), "bit_width": int(d["bit_width"]),
                   "group_size": int(d["group_size"]), "axis": int(d["axis"]), "dtype": d["dtype"],
                   "awq": None}
            if d.get("awq_scales_file"):
                out["awq"] = self._read(d["awq_scales_file"], np.float16)
            return out
        raise BundleError(f"tensor {name}: format {fmt!r} is not supported by this backend")

    def affine_int4(self, name: str) -> quant.QuantizedInt4:
        """An INT4 group-128 affine tensor in the upload layout: codes as stored, scales and
        zero-points converted to f16 (the f32 originals kept for the CPU path)."""
        t = self.tensor(name)
        if t["format"] != "affine_dequantize" or t["bit_width"] != 4:
            raise BundleError(f"tensor {name} is not INT4 affine")
        n, k = _dense_shape(t["shape"])
        gs = t["group_size"]
        if t["axis"] not in (len(t["shape"]) - 1, -1):   # the quantizer groups the last axis (quantized.rs:457)
            raise BundleError(f"tensor {name}: groups along axis {t['axis']}, the kernels group along K")
        if k % gs or gs != quant.GROUP_SIZE:
            raise BundleError(f"tensor {name}: group_size {gs} with k={k} (the kernels need 128)")
        g = k // gs
        data = t["data"]
        if data.size != n * k // 2:
            raise BundleError(f"tensor {name}: {data.size} code bytes for shape {n}x{k}")
        if t["scales"].size != n * g or t["zeros"].size != n * g:
            raise BundleError(f"tensor {name}: {t['scales'].size} scales / {t['zeros'].size} zeros for {n}x{g} groups")
        awq = t["awq"]
        if awq is not None and awq.size != k:
            raise BundleError(f"tensor {name}: {awq.size} AWQ scales for k={k}")
        s32 = t["scales"].astype(np.float32).reshape(n, g)
        z32 = t["zeros"].astype(np.float32).reshape(n, g)
        return quant.QuantizedInt4(data=data.reshape(n, k // 2).copy(), scales=to_f16_params(t["scales"]).reshape(n, g),
                                   zeros=to_f16_params(t["zeros"]).reshape(n, g), scales_f32=s32, zeros_f32=z32,
                                   awq=None if awq is None else awq.copy(), n=n, k=k, group_size=gs)

    def dense_f16(self, name: str) -> np.ndarray:
        t = self.tensor(name)
        if t["format"] != "dense":
            raise BundleError(f"tensor {name} is not dense")
        return t["data"].astype(np.float16)


def _dense_shape(shape):
    """(rows, cols) of a weight: the last dimension is K (metal/weights.rs dense_shape)."""
    if len(shape) < 2:
        raise BundleError(f"weight of shape {shape} is not a matrix")
    k = int(shape[-1])
    return int(np.prod(shape[:-1])), k


def write_bundle(path: str, config: dict, tensors: dict, n_bits: int = 4):
    """Write a bundle in the layout of write_gpu_bundle (ironmill-compile/src/gpu/bundle.rs:
    51-296) for dense tensors (numpy arrays) and INT4 affine tensors (quant.QuantizedInt4,
    written with their f32 scales and zero-points, as the quantizer produces them)."""
    wdir = os.path.join(path, "weights")
    os.makedirs(wdir, exist_ok=True)
    entries, methods = {}, set()
    for name, t in tensors.items():
        s = sanitize(name)
        if isinstance(t, quant.QuantizedInt4):
            methods.add("affine")
            files = {"quantized_data_file": f"weights/{s}.qdata", "scales_file": f"weights/{s}.scale",
                     "zeros_file": f"weights/{s}.zeros"}
            with open(os.path.join(path, files["quantized_data_file"]), "wb") as f:
                f.write(np.ascontiguousarray(t.data).tobytes())
            with open(os.path.join(path, files["scales_file"]), "wb") as f:
                f.write(np.ascontiguousarray(t.scales_f32, np.float32).tobytes())
            with open(os.path.join(path, files["zeros_file"]), "wb") as f:
                f.write(np.ascontiguousarray(t.zeros_f32, np.float32).tobytes())
            e = dict(files, shape=[t.n, t.k], bit_width=4, group_size=t.group_size, axis=1, dtype="uint8",
                     scale_dtype="float32", zero_point_dtype="float32")
            if t.awq is not None:
                e["awq_scales_file"] = f"weights/{s}.awq"
                with open(os.path.join(path, e["awq_scales_file"]), "wb") as f:
                    f.write(np.ascontiguousarray(t.awq, np.float16).tobytes())
            entries[name] = dict(format="affine_dequantize", **e)
        else:
            a = np.ascontiguousarray(t)
            dt = next((k for k, v in _DTYPES.items() if np.dtype(v) == a.dtype), None)
            if dt is None:
                raise BundleError(f"tensor {name}: dtype {a.dtype} has no manifest name")
            rel = f"weights/{s}.bin"
            with open(os.path.join(path, rel), "wb") as f:
                f.write(a.tobytes())
            entries[name] = {"format": "dense", "file": rel, "shape": list(a.shape), "dtype": dt}
    method = "none" if not methods else (methods.pop() if len(methods) == 1 else "mixed")
    manifest = {"format_version": FORMAT_VERSION, "model_config": config,
                "quantization": {"method": method, "n_bits": n_bits, "seed": 42, "min_elements": 1024},
                "tensors": entries}
    with open(os.path.join(path, "manifest.json"), "w") as f:
        json.dump(manifest, f, indent=2)


def load_decoder(dev, bundle: GpuBundle, *, max_seq_len: int, batch: int = 1, kv_cache: str = "turboquant",
                 tq_seed: int = 42, rotary_dim: int = 0, use_gelu: bool = False) -> ops.Decoder:
    """A decoder over the bundle's weights, named as load_model_weights walks them
    (weight_loading.rs:162-300): model.embed_tokens, model.layers.{i}.{input_layernorm,
    self_attn.{q,k,v,o}_proj, self_attn.{q,k}_norm, post_attention_layernorm,
    mlp.{gate,up,down}_proj}, model.norm, lm_head (or the tied INT4 embedding).
    AWQ vectors with equal contents share one device buffer, so projections that read one
    activation run as one launch."""
    c = bundle.config
    d = ops.Decoder(dev, hidden_size=c["hidden_size"], intermediate_size=c["intermediate_size"],
                    num_layers=c["num_hidden_layers"], num_heads=c["num_attention_heads"],
                    num_kv_heads=c["num_key_value_heads"], head_dim=c["head_dim"], vocab_size=c["vocab_size"],
                    max_seq_len=max_seq_len, batch=batch, rotary_dim=rotary_dim, rms_eps=float(c["rms_norm_eps"]),
                    rope_theta=float(c["rope_theta"]), use_gelu=use_gelu, kv_cache=kv_cache, tq_seed=tq_seed)
    awq_bufs = {}
    keep = []

    def weight(name):
        q = bundle.affine_int4(name)
        awq = None
        if q.awq is not None:
            key = q.awq.tobytes()
            if key not in awq_bufs:
                awq_bufs[key] = dev.upload(q.awq)
            awq = awq_bufs[key]
        w = ops.AffineQuantizedWeight.from_pointers(dev.upload(q.data), dev.upload(q.scales), dev.upload(q.zeros),
                                                    awq, q.n, q.k)
        keep.append(w)
        return w

    def dense(name):
        b = dev.upload(bundle.dense_f16(name))
        keep.append(b)
        return b

    for i in range(c["num_hidden_layers"]):
        p = f"model.layers.{i}"
        qn, kn = f"{p}.self_attn.q_norm.weight", f"{p}.self_attn.k_norm.weight"
        d.set_layer(i, input_norm=dense(f"{p}.input_layernorm.weight"),
                    post_attn_norm=dense(f"{p}.post_attention_layernorm.weight"),
                    q_norm=dense(qn) if bundle.has_tensor(qn) else None,
                    k_norm=dense(kn) if bundle.has_tensor(kn) else None,
                    q_proj=weight(f"{p}.self_attn.q_proj.weight"), k_proj=weight(f"{p}.self_attn.k_proj.weight"),
                    v_proj=weight(f"{p}.self_attn.v_proj.weight"), o_proj=weight(f"{p}.self_attn.o_proj.weight"),
                    gate_proj=weight(f"{p}.mlp.gate_proj.weight"), up_proj=weight(f"{p}.mlp.up_proj.weight"),
                    down_proj=weight(f"{p}.mlp.down_proj.weight"))
    lm_name = "lm_head.weight"
    if not bundle.has_tensor(lm_name) and c.get("tie_word_embeddings"):
        lm_name = "model.embed_tokens.weight"
    emb_desc = bundle.tensors.get("model.embed_tokens.weight", {})
    if emb_desc.get("format") == "affine_dequantize":
        raise BundleError("an INT4 embedding table needs a dense copy for the lookup; store it dense")
    d.set_model(dense("model.embed_tokens.weight"), dense("model.norm.weight"), weight(lm_name))
    d._keep["bundle"] = (keep, awq_bufs)
    return d


__all__ = ["GpuBundle", "BundleError", "write_bundle", "load_decoder", "sanitize", "to_f16_params"]

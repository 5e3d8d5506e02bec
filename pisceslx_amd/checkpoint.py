"""Reference checkpoint -> packed expert format: offline converter and loader.

The reference loads a raw state dict from ``.pt`` / ``.bin`` / ``.safetensors`` files with
``torch.load(..., weights_only=True)``, unwrapping ``model_state_dict`` / ``model`` /
``state_dict`` (tools/infer/core.py:216-227). A MoE layer's keys sit under a module prefix
(``...mlp.`` of a hybrid block, model/core/hybrid.py:1103, :1210):
``experts.{e}.{gate,up,down}_proj.*``, ``shared_experts.{s}.expert.{gate,up,down}_proj.*``,
``shared_expert_weight`` and ``router.*`` (model/moe/layer.py:665-705).

An expert matrix may be stored

* in full precision: ``<name>.weight``;
* by the reference quantizer (``YvQuantizer.quantize_model`` replaces the Linear with
  ``_YvQuantizedLinear``, model/utils/quantization.py:397-413, :486-496): ``<name>.q_weight``
  (int8 codes), ``<name>.scale``, ``<name>.zero_point``, dequantized as
  ``(q_weight - zero_point) * scale`` in fp32 — exactly the weight that module's forward uses;
* as a block-wise INT4 state (``PiscesLxBlockWiseINT4Quantizer``,
  opss/quantize/methods.py:875-960): codes 0..15 per element, one fp32 scale and int32 zero
  point per flat block, dequantized ``(q - zp) * scale`` block by block
  (:func:`dequantize_blockwise_int4`).

Conversion dequantizes each matrix to fp32 as the reference would and packs it into the
build's format (quant.py), one expert at a time (bounded memory); it is deterministic — the
same input gives the same bytes. The packed file is a safetensors file: ``experts.*`` (the
packed stack), ``router.*`` and ``shared_expert_weight`` (as in the source), and metadata with
the layer shape and format. :func:`load_packed` reads it straight to the device.

Command line::

    python -m pisceslx_amd.checkpoint list SRC
    python -m pisceslx_amd.checkpoint convert SRC DST --prefix model.layers.3.mlp. --format int8
"""
from __future__ import annotations

import argparse
import json
import os
import re
from dataclasses import dataclass
from typing import Dict, List, Optional

import torch

from .quant import FORMAT_BY_NAME, FORMAT_NAMES, ExpertPacker, PackedExperts

PACKED_VERSION = "2"  # 2: expert matrices in 16-row x 64-column blocks (quant.block_matrix)
_UNWRAP_KEYS = ("model_state_dict", "model", "state_dict")


# ------------------------------------------------------------------ reading
class StateSource:
    """Lazy read access to a checkpoint's tensors (safetensors: per key; torch: memory-mapped)."""

    def __init__(self, path: str):
        self.path = path
        if path.endswith(".safetensors"):
            from safetensors import safe_open
            self._st = safe_open(path, framework="pt", device="cpu")
            self._keys = list(self._st.keys())
            self._sd = None
        else:
            try:
                raw = torch.load(path, map_location="cpu", weights_only=True, mmap=True)
            except RuntimeError:  # not a zip-format checkpoint: no memory map
                raw = torch.load(path, map_location="cpu", weights_only=True)
            if isinstance(raw, dict):
                for k in _UNWRAP_KEYS:
                    if isinstance(raw.get(k), dict):
                        raw = raw[k]
                        break
            if not isinstance(raw, dict):
                raise ValueError(f"{path}: no state dict found")
            self._sd = {k: v for k, v in raw.items() if isinstance(v, torch.Tensor)}
            self._keys = list(self._sd.keys())
            self._st = None
        self._keyset = set(self._keys)

    def keys(self) -> List[str]:
        return self._keys

    def __contains__(self, key: str) -> bool:
        return key in self._keyset

    def get(self, key: str) -> torch.Tensor:
        if self._sd is not None:
            return self._sd[key]
        return self._st.get_tensor(key)


def find_moe_layers(keys) -> List[str]:
    """Module prefixes of the MoE layers in a checkpoint (those holding ``experts.0.gate_proj``)."""
    pat = re.compile(r"^(.*?)experts\.0\.gate_proj\.(weight|q_weight)$")
    out = []
    for k in keys:
        m = pat.match(k)
        if m and not m.group(1).endswith("shared_"):
            out.append(m.group(1))
    return sorted(set(out))


# ------------------------------------------------------------------ dequantization
def dequantize_quantized_linear(q_weight: torch.Tensor, scale: torch.Tensor,
                                zero_point: torch.Tensor) -> torch.Tensor:
    """``_YvQuantizedLinear`` weight: ``(q_weight.float() - zero_point) * scale`` (fp32,
    model/utils/quantization.py:494-496; scale / zero point broadcast: [1, in] per channel,
    scalar per tensor)."""
    return (q_weight.float() - zero_point.float()) * scale.float()


def dequantize_blockwise_int4(state: Dict[str, torch.Tensor]) -> torch.Tensor:
    """``PiscesLxBlockWiseINT4Quantizer.dequantize`` (opss/quantize/methods.py:927-960): the
    flattened codes in blocks of ``block_size``, ``(q - zero_points[b]) * scales[b]``."""
    q = state["quantized"].flatten().float()
    scales = state["scales"].float().flatten()
    zps = state["zero_points"].float().flatten()
    bs = int(state.get("block_size", 128))
    shape = state.get("original_shape", state["quantized"].shape)
    n = q.numel()
    nb = scales.numel()
    if nb * bs < n:
        raise ValueError(f"{nb} blocks of {bs} do not cover {n} elements")
    idx = torch.arange(n) // bs
    return ((q - zps[idx]) * scales[idx]).view(tuple(shape))


def linear_weight(src, name: str) -> torch.Tensor:
    """fp32 [out, in] weight of the Linear ``name`` in a state source or dict."""
    get = src.get if isinstance(src, StateSource) else src.__getitem__
    if f"{name}.weight" in src:
        return get(f"{name}.weight").float()
    if f"{name}.q_weight" in src:
        return dequantize_quantized_linear(get(f"{name}.q_weight"), get(f"{name}.scale"),
                                           get(f"{name}.zero_point"))
    raise KeyError(f"{name}: neither .weight nor .q_weight/.scale/.zero_point in the checkpoint")


# ------------------------------------------------------------------ conversion
def _count(keys, prefix: str, part: str) -> int:
    pat = re.compile(re.escape(prefix + part) + r"\.(\d+)\.")
    ids = {int(m.group(1)) for k in keys for m in [pat.match(k)] if m}
    if ids and ids != set(range(len(ids))):
        raise ValueError(f"{prefix}{part}: indices {sorted(ids)} are not 0..n-1")
    return len(ids)


def convert_layer(src, prefix: str, weight_format: str, device="cpu"):
    """Pack one MoE layer of a checkpoint. Returns (PackedExperts, router_sd, shared_weight)."""
    if not isinstance(src, StateSource) and not isinstance(src, dict):
        src = StateSource(src)
    keys = src.keys()
    E = _count(keys, prefix, "experts")
    S = _count(keys, prefix, "shared_experts")
    if E == 0:
        raise ValueError(f"no experts under prefix {prefix!r}")
    fmt = FORMAT_BY_NAME[weight_format]
    name = lambda i, m: (f"{prefix}experts.{i}.{m}_proj" if i < E
                         else f"{prefix}shared_experts.{i - E}.expert.{m}_proj")
    wg0 = linear_weight(src, name(0, "gate"))
    F, H = wg0.shape
    pk = ExpertPacker(fmt, E, S, H, F, device)
    for i in range(E + S):
        wg = wg0 if i == 0 else linear_weight(src, name(i, "gate"))
        wu = linear_weight(src, name(i, "up"))
        wd = linear_weight(src, name(i, "down"))
        if wg.shape != (F, H) or wu.shape != (F, H) or wd.shape != (H, F):
            raise ValueError(f"expert {i}: shapes {tuple(wg.shape)}, {tuple(wu.shape)}, "
                             f"{tuple(wd.shape)} do not match [{F}, {H}] / [{H}, {F}]")
        pk.set(i, wg, wu, wd)
    get = src.get if isinstance(src, StateSource) else src.__getitem__
    rp = prefix + "router."
    router = {k[len(rp):]: get(k).clone() for k in keys if k.startswith(rp)}
    sw = get(prefix + "shared_expert_weight").clone() if (prefix + "shared_expert_weight") in src else None
    return pk.packed, router, sw


_ST_DTYPES = {torch.float32: "F32", torch.bfloat16: "BF16", torch.float16: "F16",
              torch.int8: "I8", torch.uint8: "U8", torch.int32: "I32", torch.int64: "I64",
              torch.bool: "BOOL"}


def save_safetensors(tensors: Dict[str, torch.Tensor], path: str, metadata: Dict[str, str]) -> None:
    """A safetensors file with a canonical header (keys sorted, data in key order, header
    padded to 8 bytes), so the same tensors and metadata always give the same bytes (the
    safetensors library writes its metadata map in hash order)."""
    import struct
    names = sorted(tensors)
    header = {"__metadata__": {k: str(metadata[k]) for k in sorted(metadata)}}
    off = 0
    blobs = []
    for n in names:
        t = tensors[n].detach().contiguous().cpu()
        if t.dtype not in _ST_DTYPES:
            raise ValueError(f"{n}: dtype {t.dtype} has no safetensors code here")
        b = t.view(torch.uint8).numpy().tobytes() if t.numel() else b""
        header[n] = {"dtype": _ST_DTYPES[t.dtype], "shape": list(t.shape),
                     "data_offsets": [off, off + len(b)]}
        off += len(b)
        blobs.append(b)
    h = json.dumps(header, separators=(",", ":")).encode()
    h += b" " * ((8 - len(h) % 8) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)


def convert(src_path: str, dst_path: str, prefix: str, weight_format: str) -> Dict[str, str]:
    """Write the packed safetensors file of one MoE layer; returns its metadata."""
    src = StateSource(src_path)
    packed, router, sw = convert_layer(src, prefix, weight_format)
    tensors = {}
    for n in ("w_gate", "w_up", "w_down", "s_gate", "s_up", "s_down"):
        t = getattr(packed, n)
        if t is not None:
            tensors["experts." + n] = t.contiguous()
    for k, v in router.items():
        tensors["router." + k] = v.contiguous()
    if sw is not None:
        tensors["shared_expert_weight"] = sw.contiguous()
    meta = {"pisceslx_amd.packed": PACKED_VERSION, "format": FORMAT_NAMES[packed.format],
            "num_routed": str(packed.num_routed), "num_shared": str(packed.num_shared),
            "hidden": str(packed.hidden), "ffn": str(packed.ffn), "prefix": prefix,
            "source": os.path.basename(src_path)}
    tmp = dst_path + ".tmp"
    save_safetensors(tensors, tmp, meta)
    os.replace(tmp, dst_path)
    return meta


@dataclass
class PackedLayer:
    experts: PackedExperts
    router: Dict[str, torch.Tensor]
    shared_expert_weight: Optional[torch.Tensor]
    meta: Dict[str, str]


def load_packed(path: str, device="cuda") -> PackedLayer:
    """Read a packed file written by :func:`convert` onto ``device``."""
    from safetensors import safe_open
    from safetensors.torch import load_file
    with safe_open(path, framework="pt", device="cpu") as f:
        meta = dict(f.metadata() or {})
    if meta.get("pisceslx_amd.packed") != PACKED_VERSION:
        raise ValueError(f"{path}: not a packed expert file of layout version {PACKED_VERSION} "
                         f"(found {meta.get('pisceslx_amd.packed')}); convert the checkpoint again")
    t = load_file(path, device=str(device))
    experts = PackedExperts(FORMAT_BY_NAME[meta["format"]], int(meta["num_routed"]),
                            int(meta["num_shared"]), int(meta["hidden"]), int(meta["ffn"]),
                            t["experts.w_gate"], t["experts.w_up"], t["experts.w_down"],
                            t.get("experts.s_gate"), t.get("experts.s_up"), t.get("experts.s_down"))
    if experts.format == FORMAT_BY_NAME["int4"]:
        from .quant import check_int4_scales
        for name in ("s_gate", "s_up", "s_down"):
            check_int4_scales(getattr(experts, name), f"{path}: experts.{name}")
    router = {k[len("router."):]: v for k, v in t.items() if k.startswith("router.")}
    return PackedLayer(experts, router, t.get("shared_expert_weight"), meta)


# ------------------------------------------------------------------ command line
def main(argv=None) -> int:
    ap = argparse.ArgumentParser(prog="python -m pisceslx_amd.checkpoint")
    sub = ap.add_subparsers(dest="cmd", required=True)
    ls = sub.add_parser("list", help="list the MoE layer prefixes of a checkpoint")
    ls.add_argument("src")
    cv = sub.add_parser("convert", help="pack one MoE layer into a safetensors file")
    cv.add_argument("src")
    cv.add_argument("dst")
    cv.add_argument("--prefix", required=True)
    cv.add_argument("--format", required=True, choices=sorted(FORMAT_BY_NAME))
    args = ap.parse_args(argv)
    if args.cmd == "list":
        for p in find_moe_layers(StateSource(args.src).keys()):
            print(p)
        return 0
    meta = convert(args.src, args.dst, args.prefix, args.format)
    print(json.dumps(meta, sort_keys=True))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())

"""Seeded synthetic EXL3 packs (numpy): the benchmark's input recipe, in the reference pack's layout.

Recipe: trellis = uniform random u16 (every bit pattern decodes: the tail-biting reader needs no encoder), suh / svh =
fp16(+-|N(1, 0.1)|) (signs and channel scales folded into one F16 vector per side, as the reference converter stores
them: tools/convert_trunk_enc.py:137-171), router rows bf16 N(0, 1/hid) so x ~ N(0,1) gives logits ~ N(0,1),
activations bf16-representable N(0,1).

Tensor names follow the reference pack (models/flash_next/layer.mm:180-196):
    <pre>gate.weight, <pre>shared_expert_gate.weight,
    <pre>switch_mlp.{gate,up,down}_proj.{trellis,suh,svh}, <pre>shared_expert.{gate,up,down}_proj.{trellis,suh,svh}
    or, for the 8-bit affine shared expert, <pre>shared_expert.{gate,up,down}_proj.{weight,scales,biases}
"""
import json
import struct
from pathlib import Path

import numpy as np


def scales(rng, *shape):
    m = np.abs(rng.normal(1.0, 0.1, shape))
    s = np.where(rng.integers(0, 2, shape) == 1, -1.0, 1.0)
    return (m * s).astype(np.float16)


def bf16(x):
    u = np.ascontiguousarray(x, np.float32).view(np.uint32)
    return ((u + np.uint32(0x7FFF) + ((u >> 16) & np.uint32(1))) >> 16).astype(np.uint16)


def bf16_values(rng, *shape):
    """N(0,1) rounded to bf16, returned as f32"""
    return (bf16(rng.standard_normal(shape).astype(np.float32)).astype(np.uint32) << 16).view(np.float32)


def linear(rng, inp, out, K, lead=()):
    """(trellis U16 [*lead, in/16, out/16, 16K], suh F16 [*lead, in], svh F16 [*lead, out])"""
    t = rng.integers(0, 1 << 16, (*lead, inp // 16, out // 16, 16 * K), dtype=np.uint16)
    return t, scales(rng, *lead, inp), scales(rng, *lead, out)


def q8_linear(rng, inp, out, group=128):
    """8-bit affine (MLX layout, the reference's Q8): weight U32 [out, in/4] (uniform bytes, row-major), scales and
    biases bf16 bits [out, in/group]: scale = |N(1, 0.1)| / (74 sqrt(in)) (a uniform byte's deviation is ~74), bias =
    -127.5 scale, so the weights have mean ~0 and variance ~1/in"""
    wb = rng.integers(0, 256, (out, inp), dtype=np.uint8)
    sc = bf16(np.abs(rng.normal(1.0, 0.1, (out, inp // group))).astype(np.float32) / np.float32(74 * np.sqrt(inp)))
    bi = bf16(np.float32(-127.5) * (sc.astype(np.uint32) << 16).view(np.float32))
    return wb.view(np.uint32).reshape(out, inp // 4), sc, bi


def moe_layer(seed, hid=2048, inter=512, ne=512, topk=10, K=5, shared=True, Ks=None, sgate=False):
    """dict of numpy arrays for ne_moe_create / the oracle (keys as ijah_amd.engine.Engine.moe_create).
    shared: False, True (an EXL3 shared expert of Ks bits) or "q8" (the reference's 8-bit affine g128 one)."""
    rng = np.random.default_rng(seed)
    Ks = Ks or K
    w = dict(hid=hid, inter=inter, ne=ne, topk=topk, K=K, Ks=Ks if shared is True else 0)
    w["router"] = bf16(rng.standard_normal((ne, hid)).astype(np.float32) / np.float32(np.sqrt(hid)))
    if sgate:
        w["sgate"] = bf16(rng.standard_normal(hid).astype(np.float32) / np.float32(np.sqrt(hid)))
    for p, (i, o) in (("gate", (hid, inter)), ("up", (hid, inter)), ("down", (inter, hid))):
        t, su, sv = linear(rng, i, o, K, (ne,))
        w[f"{p}.trellis"], w[f"{p}.suh"], w[f"{p}.svh"] = t, su, sv
    if shared == "q8":
        for p, (i, o) in (("sq8_gate", (hid, inter)), ("sq8_up", (hid, inter)), ("sq8_down", (inter, hid))):
            w[f"{p}.weight"], w[f"{p}.scales"], w[f"{p}.biases"] = q8_linear(rng, i, o)
        w["qgroup"] = 128
    elif shared:
        for p, (i, o) in (("sgate_proj", (hid, inter)), ("sup_proj", (hid, inter)), ("sdown_proj", (inter, hid))):
            t, su, sv = linear(rng, i, o, Ks)
            w[f"{p}.trellis"], w[f"{p}.suh"], w[f"{p}.svh"] = t, su, sv
    return w


PACK_NAMES = {"gate": "switch_mlp.gate_proj", "up": "switch_mlp.up_proj", "down": "switch_mlp.down_proj",
              "sgate_proj": "shared_expert.gate_proj", "sup_proj": "shared_expert.up_proj",
              "sdown_proj": "shared_expert.down_proj", "sq8_gate": "shared_expert.gate_proj",
              "sq8_up": "shared_expert.up_proj", "sq8_down": "shared_expert.down_proj"}


def moe_tensors(w, prefix):
    """pack tensor name -> array for a moe_layer dict"""
    t = {prefix + "gate.weight": w["router"]}
    if w.get("sgate") is not None:
        t[prefix + "shared_expert_gate.weight"] = w["sgate"].reshape(1, -1)
    for k, v in w.items():
        if not isinstance(v, np.ndarray) or "." not in k:
            continue
        p, f = k.split(".")
        t[f"{prefix}{PACK_NAMES[p]}.{f}"] = v
    return t


_ST = {np.dtype(np.uint16): "U16", np.dtype(np.float16): "F16", np.dtype(np.float32): "F32",
       np.dtype(np.uint32): "U32", np.dtype(np.int32): "I32", np.dtype(np.uint8): "U8"}


def write_safetensors(path, tensors, bf16_names=(), pad_header_to=None):
    """Writes a safetensors file; arrays named in bf16_names are stored as BF16 (uint16 bits)."""
    hdr, off, blobs = {}, 0, []
    for name in sorted(tensors):
        a = np.ascontiguousarray(tensors[name])
        dt = "BF16" if name in bf16_names else _ST[a.dtype]
        hdr[name] = {"dtype": dt, "shape": list(a.shape), "data_offsets": [off, off + a.nbytes]}
        blobs.append(a)
        off += a.nbytes
    h = json.dumps(hdr, separators=(",", ":")).encode()
    if pad_header_to:
        h += b" " * ((-len(h) - 8) % pad_header_to)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for a in blobs:
            f.write(a.tobytes())


def write_moe_pack(directory, w, layer=0, extra=None, shards=1):
    """A pack directory with one MoE layer (plus `extra` tensors): config.json + shard files."""
    d = Path(directory)
    d.mkdir(parents=True, exist_ok=True)
    prefix = f"language_model.model.layers.{layer}.mlp."
    t = moe_tensors(w, prefix)
    if extra:
        t.update(extra)
    bfn = {prefix + "gate.weight", prefix + "shared_expert_gate.weight"} | \
        {n for n in t if n.endswith(".scales") or n.endswith(".biases")}
    names = sorted(t)
    per = (len(names) + shards - 1) // shards
    for i in range(shards):
        part = {n: t[n] for n in names[i * per:(i + 1) * per]}
        write_safetensors(d / f"model-{i:05d}-of-{shards:05d}.safetensors", part, bfn)
    cfg = {"expert_quant": {"codebook": "mcg", "window": 15, "layer_k": w["K"]}, "hidden_size": w["hid"],
           "moe_intermediate_size": w["inter"], "num_experts": w["ne"], "num_experts_per_tok": w["topk"]}
    (d / "config.json").write_text(json.dumps(cfg))
    return prefix

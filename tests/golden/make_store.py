"""Writes weight stores in the two on-disk forms qf_store_open reads.

- safetensors: an 8-byte little-endian header length, a JSON header (padded
  with spaces to a multiple of 8) mapping each tensor name to its dtype, shape
  and [begin, end) byte range in the data region, then the data region. Data
  may be left as holes (sparse files) when only the index matters.
- the reference engine's index (ocho/amd_server/qwenflash.h:12-30,
  reader.cpp:15-61): shards.txt (one shard path per line) and manifest.bin
  (512-byte records: name[256], QfRec, padding), packed field by field here.

Tensor names and shapes follow the reference checkpoint
(ocho/engine_spark/model.cpp:238-250, :380-395; qf_hip4_stage.hip:628-641):
routed experts as NVFP4 (packed e2m1 [rows][in/2] U8, e4m3 block scales
[rows][in/16] F8_E4M3, weight_scale_2 F32 scalar), the router, the shared
expert and its gate vector as BF16.

Command line: python make_store.py OUT_DIR [--hidden 2048 --inter 512
--experts 512 --layer 0 --seed 7 --shards 3 --sparse] writes one synthetic
layer, its routed experts made with the test oracle's counter-based generator
(the same bytes qfm_arena_generate produces on the device)."""
import argparse
import json
import os
import struct
import sys

import numpy as np

DTYPE_SIZE = {"BF16": 2, "F32": 4, "U8": 1, "F8_E4M3": 1, "I64": 8, "F16": 2, "I8": 1, "I32": 4, "F64": 8,
              "F8_E5M2": 1, "I16": 2, "U16": 2, "U32": 4, "U64": 8, "BOOL": 1}
DTYPE_CODE = {"BF16": 1, "F32": 2, "U8": 3, "F8_E4M3": 4, "I64": 5, "F16": 6, "I8": 7, "I32": 8, "F64": 9,
              "F8_E5M2": 10, "I16": 11, "U16": 12, "U32": 13, "U64": 14, "BOOL": 15}
PROJ = ("gate_proj", "up_proj", "down_proj")
PFX = "model.language_model.layers.{L}.mlp"


def _count(shape):
    n = 1
    for d in shape:
        n *= int(d)
    return n


def write_safetensors(path, tensors, metadata=None):
    """tensors: list of (name, dtype, shape, data); data is bytes-like of the
    exact size, or None for zero bytes left as a hole. Returns {name:
    (absolute data offset, nbytes)}."""
    header, spans, off = {}, {}, 0
    for name, dt, shape, data in tensors:
        n = _count(shape) * DTYPE_SIZE[dt]
        if data is not None and len(memoryview(data).cast("B")) != n:
            raise ValueError(f"{name}: {len(memoryview(data).cast('B'))} bytes for shape {shape} {dt}")
        header[name] = {"dtype": dt, "shape": [int(d) for d in shape], "data_offsets": [off, off + n]}
        spans[name] = (off, n)
        off += n
    if metadata:
        header["__metadata__"] = metadata
    hb = json.dumps(header, separators=(",", ":")).encode()
    hb += b" " * (-len(hb) % 8)
    base = 8 + len(hb)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hb)))
        f.write(hb)
        for name, dt, shape, data in tensors:
            if data is None:
                f.seek(spans[name][1], 1)
            else:
                f.write(memoryview(data).cast("B"))
        f.truncate(base + off)
    return {k: (base + o, n) for k, (o, n) in spans.items()}


def manifest_record(name, file_idx, dtype_code, ne, data_off, nbytes, scale2_off=0, input_off=0, scale2_file=0,
                    input_file=0, flags=0):
    """One 512-byte QfEntry: name[256] NUL-padded, then QfRec {u32 file_idx,
    u32 dtype, u64 ne[4], u64 data_off, u64 nbytes, u64 scale2_off, u64
    input_off, u32 scale2_file, u32 input_file, u32 flags, 4 pad}, then 168 pad."""
    b = name.encode()
    if len(b) >= 256:
        raise ValueError("name too long")
    ne4 = list(ne) + [1] * (4 - len(ne))
    rec = b.ljust(256, b"\0") + struct.pack("<II4QQQQQIII4x", file_idx, dtype_code, *ne4, data_off, nbytes,
                                            scale2_off, input_off, scale2_file, input_file, flags)
    rec += b"\0" * (512 - len(rec))
    assert len(rec) == 512
    return rec


def write_manifest(dirpath, shard_paths, records):
    os.makedirs(dirpath, exist_ok=True)
    with open(os.path.join(dirpath, "shards.txt"), "w") as f:
        for p in shard_paths:
            f.write(p + "\n")
    with open(os.path.join(dirpath, "manifest.bin"), "wb") as f:
        for r in records:
            f.write(r)


def manifest_from_safetensors(dirpath, shard_paths):
    """The reference index for existing safetensors shards: one record per
    tensor, data_off absolute in its shard file."""
    recs = []
    for i, p in enumerate(shard_paths):
        with open(p, "rb") as f:
            n = struct.unpack("<Q", f.read(8))[0]
            hdr = json.loads(f.read(n))
        for name, meta in hdr.items():
            if name == "__metadata__":
                continue
            b, e = meta["data_offsets"]
            recs.append(manifest_record(name, i, DTYPE_CODE[meta["dtype"]], list(reversed(meta["shape"])) or [1],
                                        8 + n + b, e - b))
    write_manifest(dirpath, shard_paths, recs)


def expert_name(layer, e, proj, suffix):
    return f"{PFX.format(L=layer)}.experts.{e}.{proj}.{suffix}"


def expert_tensors(layer, e, H, I, w=None, s=None, s2=(0.01, 0.01, 0.01)):
    """The 9 checkpoint tensors of routed expert e. w / s: three packed-weight
    / block-scale byte arrays (gate, up, down), or None for holes."""
    out = []
    for p, proj in enumerate(PROJ):
        rows, cols = (H, I) if p == 2 else (I, H)
        out.append((expert_name(layer, e, proj, "weight"), "U8", (rows, cols // 2), None if w is None else w[p]))
        out.append((expert_name(layer, e, proj, "weight_scale"), "F8_E4M3", (rows, cols // 16),
                    None if s is None else s[p]))
        out.append((expert_name(layer, e, proj, "weight_scale_2"), "F32", (), np.float32(s2[p]).tobytes()))
    return out


def dense_tensors(layer, H, I, E, router=None, shared=None, gate_vec=None):
    """Router [E][H], shared expert gate/up [I][H] and down [H][I], shared gate
    [1][H], all BF16 (uint16 bit arrays, or None for holes)."""
    P = PFX.format(L=layer)
    sh = shared if shared is not None else (None, None, None)
    return [(f"{P}.gate.weight", "BF16", (E, H), router),
            (f"{P}.shared_expert.gate_proj.weight", "BF16", (I, H), sh[0]),
            (f"{P}.shared_expert.up_proj.weight", "BF16", (I, H), sh[1]),
            (f"{P}.shared_expert.down_proj.weight", "BF16", (H, I), sh[2]),
            (f"{P}.shared_expert_gate.weight", "BF16", (1, H), gate_vec)]


def bf16_rne(a):
    """fp32 -> bf16 bits, round to nearest even (finite inputs)."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def synthetic_layer(out_dir, H, I, E, layer, seed, shards=3, sparse=False):
    """One layer: experts from the oracle generator (tensors 11-16, the device
    generator's NVFP4 arena for (seed, layer); weight_scale_2 = 0.01), dense
    tensors from generator Gaussians rounded to BF16. Returns the shard paths."""
    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    import _oracle as orc
    os.makedirs(out_dir, exist_ok=True)
    IH = I * H
    per = (E + shards - 1) // shards
    paths = []
    for sh in range(shards):
        ts = []
        for e in range(sh * per, min(E, (sh + 1) * per)):
            if sparse:
                ts += expert_tensors(layer, e, H, I)
                continue
            w = [orc.fill("fp4byte", seed, layer, t, e * IH // 2, IH // 2) for t in (orc.T_FG, orc.T_FU, orc.T_FD)]
            s = [orc.fill("e4m3scale", seed, layer, t, e * IH // 16, IH // 16) for t in (orc.T_FSG, orc.T_FSU, orc.T_FSD)]
            ts += expert_tensors(layer, e, H, I, w, s)
        if sh == shards - 1:
            if sparse:
                ts += dense_tensors(layer, H, I, E)
            else:
                g = lambda t, n, sc: bf16_rne(orc.fill("gauss", seed, layer, t, 0, n, sc))
                ts += dense_tensors(layer, H, I, E, router=g(orc.T_ROUTER, E * H, 0.02),
                                    shared=(g(101, IH, 0.05), g(102, IH, 0.05), g(103, IH, 0.05)),
                                    gate_vec=g(orc.T_SHGATE, H, 0.02))
        p = os.path.join(out_dir, f"model-{sh + 1:05d}-of-{shards:05d}.safetensors")
        write_safetensors(p, ts, metadata={"format": "pt"})
        paths.append(p)
    return paths


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("out_dir")
    ap.add_argument("--hidden", type=int, default=2048)
    ap.add_argument("--inter", type=int, default=512)
    ap.add_argument("--experts", type=int, default=512)
    ap.add_argument("--layer", type=int, default=0)
    ap.add_argument("--seed", type=int, default=7)
    ap.add_argument("--shards", type=int, default=3)
    ap.add_argument("--sparse", action="store_true", help="leave tensor data as holes (index checks only)")
    ap.add_argument("--manifest", action="store_true", help="also write the reference index (shards.txt, manifest.bin)")
    a = ap.parse_args()
    paths = synthetic_layer(a.out_dir, a.hidden, a.inter, a.experts, a.layer, a.seed, a.shards, a.sparse)
    if a.manifest:
        manifest_from_safetensors(os.path.join(a.out_dir, "index"), paths)
    print("\n".join(paths))


if __name__ == "__main__":
    main()

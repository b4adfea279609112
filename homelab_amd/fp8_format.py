"""The fp8-e4m3-b128 expert-record layout, and a converter to it from the reference's
on-disk format.

The reference's weight format (docs/dev/format.md; crates/oominf-format/src/lib.rs) stores
routed experts one record per (layer, expert) in experts.bin, every record of a group
sharing one record schema: an ordered list of parts (name, dtype, shape, offset, nbytes),
each part at a 256-byte offset (PART_ALIGN), the stride rounded up to 4096 (ALIGN), and
a layout tag naming the encoding; a loader that does not implement a tag refuses the
group (format.md "No silent misreads"). v0 defines the tags nvfp4-modelopt-g16 and bf16.

This module adds the tag of the FP8 kernels' records:

    fp8-e4m3-b128   parts, in order:
        gate.weight  F8_E4M3 [inter, hidden]   row-major
        gate.scale   F32     [ceil(inter / 128), ceil(hidden / 128)]
        up.weight    F8_E4M3 [inter, hidden]
        up.scale     F32     [ceil(inter / 128), ceil(hidden / 128)]
        down.weight  F8_E4M3 [hidden, inter]
        down.scale   F32     [ceil(hidden / 128), ceil(inter / 128)]
    w[r, c] = e4m3(q[r, c]) * scale[r / 128, c / 128]; per 128 x 128 block,
    scale = absmax / 448 (1 for an all-zero block) and q = e4m3(w / scale), rounded to
    nearest even and saturated at +-448 (crates/oominf-core/src/fp8.rs:5-27,52-88 with
    128 x 128 blocks).

The offsets are those of record_geometry (the OomFp8Record the C ABI takes), so a record
read verbatim into device memory is what oom_moe_decode_fp8 and oom_moe_prefill_fp8 read.

convert_model() re-lays a converted model directory: every expert group with layout bf16
(the reference's unquantised records: gate.weight, up.weight BF16 [inter, hidden],
down.weight BF16 [hidden, inter]) becomes an fp8-e4m3-b128 group, one record at a time;
other groups, dense.bin and tables.bin are copied unchanged. open_fp8_group() is the
loader side: it refuses any other layout tag and checks each record's xxh3-64.

    python -m homelab_amd.fp8_format SRC_DIR DST_DIR
"""
from __future__ import annotations

import json
import os
import shutil
import sys

import numpy as np

FORMAT_TAG = "oominf"
FORMAT_VERSION = 0
INDEX_NAME = "index.json"
EXPERTS_FILE = "experts.bin"
ALIGN = 4096
PART_ALIGN = 256
LAYOUT_FP8 = "fp8-e4m3-b128"
LAYOUT_BF16 = "bf16"
BLOCK = 128

_DTYPE_SIZE = {"BOOL": 1, "U8": 1, "I8": 1, "F8_E4M3": 1, "F8_E5M2": 1, "BF16": 2, "F16": 2, "I16": 2, "U16": 2,
               "F32": 4, "I32": 4, "U32": 4, "F64": 8, "I64": 8, "U64": 8}


class FormatError(ValueError):
    """A model directory or record this code will not read (unknown layout tag, wrong
    sizes, checksum mismatch)."""


def align_up(n: int, to: int) -> int:
    return (n + to - 1) // to * to


def checksum(data) -> str:
    """xxh3-64 as 16 lowercase hex digits (crates/oominf-format/src/lib.rs:70-72)."""
    import xxhash

    return format(xxhash.xxh3_64_intdigest(bytes(data) if not isinstance(data, (bytes, bytearray)) else data), "016x")


def record_schema(layout: str, parts) -> dict:
    """Parts laid out in order at PART_ALIGN offsets, the stride rounded up to ALIGN
    (RecordSchema::new, crates/oominf-format/src/lib.rs:157-176)."""
    off = 0
    laid = []
    for name, dtype, shape in parts:
        nbytes = _DTYPE_SIZE[dtype] * int(np.prod(shape))
        laid.append({"name": name, "dtype": dtype, "shape": [int(s) for s in shape], "offset": off, "nbytes": nbytes})
        off = align_up(off + nbytes, PART_ALIGN)
    return {"layout": layout, "parts": laid, "stride": align_up(off, ALIGN)}


def fp8_schema(hidden: int, inter: int) -> dict:
    """The fp8-e4m3-b128 record schema of an expert with this geometry."""
    nb = lambda n: (n + BLOCK - 1) // BLOCK  # noqa: E731
    return record_schema(LAYOUT_FP8, [
        ("gate.weight", "F8_E4M3", [inter, hidden]), ("gate.scale", "F32", [nb(inter), nb(hidden)]),
        ("up.weight", "F8_E4M3", [inter, hidden]), ("up.scale", "F32", [nb(inter), nb(hidden)]),
        ("down.weight", "F8_E4M3", [hidden, inter]), ("down.scale", "F32", [nb(hidden), nb(inter)]),
    ])


def _part(schema: dict, name: str) -> dict:
    for p in schema["parts"]:
        if p["name"] == name:
            return p
    raise FormatError(f"record schema ({schema['layout']}) has no part {name}")


def geometry(schema: dict):
    """The OomFp8Record of an fp8-e4m3-b128 schema (raises for any other layout)."""
    from . import Fp8Record

    if schema["layout"] != LAYOUT_FP8:
        raise FormatError(f"layout {schema['layout']!r} is not {LAYOUT_FP8!r}")
    inter, hidden = _part(schema, "gate.weight")["shape"]
    want = fp8_schema(hidden, inter)
    if want != {k: schema[k] for k in ("layout", "parts", "stride")}:
        raise FormatError("fp8-e4m3-b128 schema does not have the layout's part offsets")
    o = {p["name"]: p["offset"] for p in schema["parts"]}
    return Fp8Record(hidden, inter, o["gate.weight"], o["gate.scale"], o["up.weight"], o["up.scale"],
                     o["down.weight"], o["down.scale"])


def e4m3_rne(x) -> np.ndarray:
    """e4m3fn codes of f32 values: round to nearest even, saturating at +-448 (0x7e), NaN to
    sign | 0x7e, sign kept for zero (crates/oominf-core/src/fp8.rs:5-27). Normal codes are (e + 7) << 3 |
    (m - 8) for |x| = m 2^(e - 3), 8 <= m < 16; subnormals (|x| < 2^-6) are m for
    |x| = m 2^-9 -- both (e + 6) 8 + m with e = -6 below 2^-6, which also carries a
    mantissa that rounds up to 16 into the next exponent."""
    x = np.asarray(x, dtype=np.float32)
    sign = np.signbit(x).astype(np.uint8) << 7
    a = np.abs(x).astype(np.float64)
    a = np.minimum(np.where(np.isnan(a), 448.0, a), 448.0)  # NaN saturates like +-inf: sign | 0x7e
    _, ex = np.frexp(a)
    e = np.where(a < 2.0 ** -6, -6, ex.astype(np.int64) - 1)
    m = np.rint(a / np.exp2((e - 3).astype(np.float64)))  # exact scaling; half to even
    code = ((e + 6) * 8 + m.astype(np.int64)).astype(np.uint8)
    return code | sign


def bf16_to_f32(bits) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def quantize_blocks(w_bits) -> tuple[np.ndarray, np.ndarray]:
    """(q uint8 [n, k], scale f32 [ceil(n / 128), ceil(k / 128)]) of bf16 weights (uint16
    bits) with 128 x 128 absmax blocks: scale = absmax / 448 in f32 (1 for an all-zero
    block), q = e4m3(w / scale) with an f32 division."""
    w = bf16_to_f32(w_bits)
    n, k = w.shape
    nbr, nbc = (n + BLOCK - 1) // BLOCK, (k + BLOCK - 1) // BLOCK
    pad = np.zeros((nbr * BLOCK, nbc * BLOCK), dtype=np.float32)
    pad[:n, :k] = np.abs(w)
    # NaN-ignoring maximum from 0, as f32::max folds (an all-NaN block gets scale 1)
    amax = np.fmax.reduce(pad.reshape(nbr, BLOCK, nbc, BLOCK), axis=(1, 3), initial=np.float32(0.0))
    s = np.where(amax > 0, amax / np.float32(448.0), np.float32(1.0)).astype(np.float32)
    full = np.repeat(np.repeat(s, BLOCK, axis=0), BLOCK, axis=1)[:n, :k]
    q = e4m3_rne(w / full)
    return q, s


def convert_record(src: np.ndarray, src_schema: dict) -> np.ndarray:
    """One bf16-layout record (its stride bytes) as an fp8-e4m3-b128 record (uint8 of
    the new stride, padding zero)."""
    if src_schema["layout"] != LAYOUT_BF16:
        raise FormatError(f"convert_record reads layout {LAYOUT_BF16!r}, not {src_schema['layout']!r}")
    src = np.asarray(src, dtype=np.uint8)
    parts = {}
    for name in ("gate.weight", "up.weight", "down.weight"):
        p = _part(src_schema, name)
        if p["dtype"] != "BF16" or len(p["shape"]) != 2:
            raise FormatError(f"{name}: want a 2-D BF16 part, got {p['dtype']} {p['shape']}")
        parts[name] = src[p["offset"]:p["offset"] + p["nbytes"]].view(np.uint16).reshape(p["shape"])
    inter, hidden = parts["gate.weight"].shape
    if parts["up.weight"].shape != (inter, hidden) or parts["down.weight"].shape != (hidden, inter):
        raise FormatError("bf16 record: gate/up must be [inter, hidden] and down [hidden, inter]")
    dst_schema = fp8_schema(hidden, inter)
    out = np.zeros(dst_schema["stride"], dtype=np.uint8)
    for proj in ("gate", "up", "down"):
        q, s = quantize_blocks(parts[f"{proj}.weight"])
        pw, ps = _part(dst_schema, f"{proj}.weight"), _part(dst_schema, f"{proj}.scale")
        out[pw["offset"]:pw["offset"] + pw["nbytes"]] = q.reshape(-1)
        out[ps["offset"]:ps["offset"] + ps["nbytes"]] = s.reshape(-1).view(np.uint8)
    return out


def _read_index(model_dir: str) -> dict:
    with open(os.path.join(model_dir, INDEX_NAME)) as f:
        index = json.load(f)
    if index.get("format") != FORMAT_TAG or index.get("version") != FORMAT_VERSION:
        raise FormatError(f"unsupported format {index.get('format')} v{index.get('version')} "
                          f"(want {FORMAT_TAG} v{FORMAT_VERSION})")
    return index


def convert_model(src_dir: str, dst_dir: str) -> dict:
    """Writes dst_dir: src_dir with every bf16 expert group as fp8-e4m3-b128. Records
    stream one at a time; each new record gets its xxh3-64. Returns the new index."""
    index = _read_index(src_dir)
    os.makedirs(dst_dir, exist_ok=True)
    groups = []
    off = 0
    with open(os.path.join(src_dir, EXPERTS_FILE), "rb") as fin, \
            open(os.path.join(dst_dir, EXPERTS_FILE), "wb") as fout:
        for g in index["expert_groups"]:
            src_schema = {k: g[k] for k in ("layout", "parts", "stride")}
            convert = g["layout"] == LAYOUT_BF16
            sums = []
            new_schema = None
            for e in range(g["num_experts"]):
                fin.seek(g["offset"] + e * g["stride"])
                raw = np.frombuffer(fin.read(g["stride"]), dtype=np.uint8)
                if len(raw) != g["stride"]:
                    raise FormatError(f"layer {g['layer']} expert {e}: experts.bin is short")
                rec = convert_record(raw, src_schema) if convert else raw
                if convert and new_schema is None:
                    inter, hidden = _part(src_schema, "gate.weight")["shape"]
                    new_schema = fp8_schema(hidden, inter)
                fout.write(rec.tobytes())
                sums.append(checksum(rec.tobytes()))
            schema = new_schema if convert else src_schema
            if schema is None:  # a bf16 group with no experts
                inter, hidden = _part(src_schema, "gate.weight")["shape"]
                schema = fp8_schema(hidden, inter)
            ng = dict(g)
            ng.update(schema)
            ng["offset"] = off
            ng["xxh3"] = sums if convert else g["xxh3"]
            groups.append(ng)
            off += g["num_experts"] * schema["stride"]
    for name in ("dense.bin", "tables.bin"):
        if os.path.exists(os.path.join(src_dir, name)):
            shutil.copyfile(os.path.join(src_dir, name), os.path.join(dst_dir, name))
    for name in os.listdir(src_dir):  # config.json, tokenizer files, ...: verbatim
        if name not in (INDEX_NAME, EXPERTS_FILE, "dense.bin", "tables.bin") and \
                os.path.isfile(os.path.join(src_dir, name)):
            shutil.copyfile(os.path.join(src_dir, name), os.path.join(dst_dir, name))
    new = dict(index)
    new["expert_groups"] = groups
    new["files"] = dict(index["files"])
    new["files"]["experts"] = {"bytes": off}
    with open(os.path.join(dst_dir, INDEX_NAME), "w") as f:
        json.dump(new, f, indent=1)
    return new


class Fp8Group:
    """The fp8-e4m3-b128 records of one layer: geometry (OomFp8Record), stride, and
    record reads checked against their xxh3-64."""

    def __init__(self, model_dir: str, layer: int):
        index = _read_index(model_dir)
        found = [g for g in index["expert_groups"] if g["layer"] == layer]
        if not found:
            raise FormatError(f"no expert group for layer {layer}")
        g = found[0]
        self.geo = geometry({k: g[k] for k in ("layout", "parts", "stride")})  # refuses other tags
        self.stride = int(g["stride"])
        self.num_experts = int(g["num_experts"])
        self.offset = int(g["offset"])
        self.sums = list(g["xxh3"])
        self.path = os.path.join(model_dir, EXPERTS_FILE)
        size = os.path.getsize(self.path)
        if size != index["files"]["experts"]["bytes"]:
            raise FormatError(f"experts.bin is {size} bytes, index says {index['files']['experts']['bytes']}")

    def read(self, expert: int, verify: bool = True) -> np.ndarray:
        if not 0 <= expert < self.num_experts:
            raise FormatError(f"expert {expert} out of range ({self.num_experts} experts)")
        with open(self.path, "rb") as f:
            f.seek(self.offset + expert * self.stride)
            raw = f.read(self.stride)
        if verify and checksum(raw) != self.sums[expert]:
            raise FormatError(f"expert {expert}: checksum mismatch")
        return np.frombuffer(raw, dtype=np.uint8)


def open_fp8_group(model_dir: str, layer: int) -> Fp8Group:
    return Fp8Group(model_dir, layer)


def main(argv=None) -> int:
    argv = sys.argv[1:] if argv is None else argv
    if len(argv) != 2:
        print("usage: python -m homelab_amd.fp8_format SRC_DIR DST_DIR", file=sys.stderr)
        return 2
    idx = convert_model(argv[0], argv[1])
    n = sum(g["num_experts"] for g in idx["expert_groups"] if g["layout"] == LAYOUT_FP8)
    print(f"wrote {argv[1]}: {n} fp8-e4m3-b128 records, experts.bin {idx['files']['experts']['bytes']} bytes")
    return 0


if __name__ == "__main__":
    sys.exit(main())

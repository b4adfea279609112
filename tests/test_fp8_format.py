"""The fp8-e4m3-b128 record layout and the bf16 -> fp8 converter (homelab_amd/fp8_format.py).

Pins: the schema's part offsets equal the C ABI's record geometry (and the oracle's); the
numpy e4m3 encoder round-trips every finite code and agrees with the oracle's
e4m3_from_f32 (pinned by the reference's fp8.rs known answers) on ties, subnormals and
saturation; the block quantiser equals oracle.quantize bit for bit; a converted model
directory holds exactly the oracle's quantised records with correct xxh3-64 checksums,
copies every other group and file unchanged, and its loader refuses other layout tags
and corrupted records. The GPU test runs the decode step on converted records against
the oracle.
"""
import json
import os

import numpy as np
import pytest

import homelab_amd as hip
import oracle
from homelab_amd import fp8_format as ff


@pytest.mark.parametrize("hidden,inter", [(4096, 1536), (256, 128), (300, 200), (2560, 640)])
def test_schema_matches_record_geometry(hidden, inter):
    s = ff.fp8_schema(hidden, inter)
    g = ff.geometry(s)
    for want in (hip.record_geometry(hidden, inter), oracle.record_geometry(hidden, inter)):
        for f in ("hidden", "inter", "gate_weight", "gate_scale", "up_weight", "up_scale", "down_weight",
                  "down_scale"):
            assert getattr(g, f) == getattr(want, f), f
    assert s["stride"] == hip.record_stride(hip.record_geometry(hidden, inter))
    assert all(p["offset"] % ff.PART_ALIGN == 0 for p in s["parts"]) and s["stride"] % ff.ALIGN == 0


def test_e4m3_every_code_round_trips():
    codes = np.array([c for c in range(256) if c & 0x7f != 0x7f], dtype=np.uint8)
    vals = np.array([oracle.e4m3_to_f32(int(c)) for c in codes], dtype=np.float32)
    np.testing.assert_array_equal(ff.e4m3_rne(vals), codes)


def test_e4m3_matches_oracle_on_ties_subnormals_and_saturation():
    rng = np.random.default_rng(3)
    pos = np.array([oracle.e4m3_to_f32(c) for c in range(0x7f)], dtype=np.float64)
    mids = (pos[:-1] + pos[1:]) / 2  # exact ties between neighbouring codes
    x = np.concatenate([mids, -mids, pos, [0.0, -0.0, 448.0, 449.0, 464.0, 500.0, 1e6, -1e6, 2.0 ** -10, 2.0 ** -11,
                                          3 * 2.0 ** -11, -(2.0 ** -12), np.nan, -np.nan, np.inf, -np.inf],
                        rng.standard_normal(5000) * 40, rng.standard_normal(2000) * 0.01]).astype(np.float32)
    want = np.array([oracle.e4m3_from_f32(float(v)) for v in x], dtype=np.uint8)
    np.testing.assert_array_equal(ff.e4m3_rne(x), want)


def random_bf16(shape, seed, scale=0.02):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal(shape) * scale).astype(np.float32)
    w[::7, ::11] *= 300.0  # outliers set some blocks' absmax
    return oracle.bf16_from_f32(w)


@pytest.mark.parametrize("n,k", [(256, 384), (300, 200), (128, 128), (1, 5)])
def test_quantize_blocks_matches_oracle(n, k):
    w = random_bf16((n, k), n * 7 + k)
    w[: min(n, 128), : min(k, 128)] = 0  # an all-zero block takes scale 1
    w[-1, -1] = 0x7fc0  # a NaN: ignored by the block maximum, coded as 0x7e
    if n > 128 and k > 128:
        w[128:, 128:256] = 0xffc0  # an all-NaN block: scale 1, every code sign | 0x7e
    q, s = ff.quantize_blocks(w)
    wq, ws = oracle.quantize(w, oracle.SCALE_128X128)
    np.testing.assert_array_equal(q, wq)
    np.testing.assert_array_equal(s.reshape(-1), ws)


def write_model(d, layers):
    """A model directory in the reference's format: `layers` = [(layer, layout, records,
    parts)], records a list of uint8 arrays of the schema stride."""
    os.makedirs(d, exist_ok=True)
    groups = []
    off = 0
    with open(os.path.join(d, "experts.bin"), "wb") as f:
        for layer, layout, recs, parts in layers:
            schema = ff.record_schema(layout, parts)
            for r in recs:
                assert len(r) == schema["stride"]
                f.write(r.tobytes())
            groups.append({"layer": layer, "num_experts": len(recs), "offset": off, **schema,
                           "xxh3": [ff.checksum(r.tobytes()) for r in recs]})
            off += len(recs) * schema["stride"]
    dense = np.arange(4096, dtype=np.uint8)
    with open(os.path.join(d, "dense.bin"), "wb") as f:
        f.write(dense.tobytes())
    with open(os.path.join(d, "tables.bin"), "wb") as f:
        pass
    with open(os.path.join(d, "config.json"), "w") as f:
        f.write('{"model_type": "test"}')
    index = {"format": "oominf", "version": 0,
             "source": {"origin": "test/synthetic@0", "model_type": "test", "fingerprint": ""},
             "files": {"dense": {"bytes": 4096}, "experts": {"bytes": off}, "tables": {"bytes": 0}},
             "tensors": [{"name": "embed", "file": "dense", "dtype": "U8", "shape": [4096], "offset": 0,
                          "nbytes": 4096, "xxh3": ff.checksum(dense.tobytes())}],
             "expert_groups": groups}
    with open(os.path.join(d, "index.json"), "w") as f:
        json.dump(index, f)


def bf16_group(hidden, inter, n, seed):
    parts = [("gate.weight", "BF16", [inter, hidden]), ("up.weight", "BF16", [inter, hidden]),
             ("down.weight", "BF16", [hidden, inter])]
    schema = ff.record_schema("bf16", parts)
    recs, mats = [], []
    for e in range(n):
        g = random_bf16((inter, hidden), seed + 3 * e)
        u = random_bf16((inter, hidden), seed + 3 * e + 1)
        dn = random_bf16((hidden, inter), seed + 3 * e + 2)
        r = np.zeros(schema["stride"], dtype=np.uint8)
        for (name, _, _), m in zip(parts, (g, u, dn)):
            p = next(p for p in schema["parts"] if p["name"] == name)
            r[p["offset"]:p["offset"] + p["nbytes"]] = m.reshape(-1).view(np.uint8)
        recs.append(r)
        mats.append((g, u, dn))
    return recs, mats, parts


def oracle_record(g, u, dn):
    """The fp8-e4m3-b128 record of bf16 matrices, built from the oracle's quantiser."""
    inter, hidden = g.shape
    geo = oracle.record_geometry(hidden, inter)
    rec = np.zeros(hip.record_stride(hip.record_geometry(hidden, inter)), dtype=np.uint8)
    for m, wo, so in ((g, geo.gate_weight, geo.gate_scale), (u, geo.up_weight, geo.up_scale),
                      (dn, geo.down_weight, geo.down_scale)):
        q, s = oracle.quantize(m, oracle.SCALE_128X128)
        rec[wo:wo + q.size] = q.reshape(-1)
        rec[so:so + 4 * s.size] = s.view(np.uint8)
    return rec


def test_convert_model(tmp_path):
    src, dst = str(tmp_path / "src"), str(tmp_path / "dst")
    hidden, inter = 256, 128
    recs, mats, parts = bf16_group(hidden, inter, 3, 11)
    rng = np.random.default_rng(5)
    nv_parts = [("scalars", "F32", [64]), ("gate.weight", "U8", [64, 64])]
    nv_stride = ff.record_schema("nvfp4-modelopt-g16", nv_parts)["stride"]
    nv = [rng.integers(0, 256, nv_stride, dtype=np.uint8) for _ in range(2)]
    write_model(src, [(0, "bf16", recs, parts), (1, "nvfp4-modelopt-g16", nv, nv_parts)])
    idx = ff.convert_model(src, dst)
    g0, g1 = idx["expert_groups"]
    assert g0["layout"] == ff.LAYOUT_FP8 and g1["layout"] == "nvfp4-modelopt-g16"
    grp = ff.open_fp8_group(dst, 0)
    assert grp.num_experts == 3 and grp.stride == hip.record_stride(hip.record_geometry(hidden, inter))
    for e, (g, u, dn) in enumerate(mats):
        np.testing.assert_array_equal(grp.read(e), oracle_record(g, u, dn))
    with open(os.path.join(dst, "experts.bin"), "rb") as f:
        for e in range(2):
            f.seek(g1["offset"] + e * g1["stride"])
            np.testing.assert_array_equal(np.frombuffer(f.read(g1["stride"]), dtype=np.uint8), nv[e])
            assert g1["xxh3"][e] == ff.checksum(nv[e].tobytes())
    for name in ("dense.bin", "config.json"):
        assert open(os.path.join(src, name), "rb").read() == open(os.path.join(dst, name), "rb").read()
    assert os.path.getsize(os.path.join(dst, "experts.bin")) == idx["files"]["experts"]["bytes"]


def test_loader_refuses_other_layouts_and_corruption(tmp_path):
    src, dst = str(tmp_path / "src"), str(tmp_path / "dst")
    recs, _, parts = bf16_group(128, 128, 2, 21)
    write_model(src, [(0, "bf16", recs, parts)])
    with pytest.raises(ff.FormatError, match="not 'fp8-e4m3-b128'"):
        ff.open_fp8_group(src, 0)  # the bf16 group itself
    ff.convert_model(src, dst)
    with pytest.raises(ff.FormatError, match="no expert group"):
        ff.open_fp8_group(dst, 5)
    grp = ff.open_fp8_group(dst, 0)
    with open(os.path.join(dst, "experts.bin"), "r+b") as f:
        f.seek(grp.offset + grp.stride + 17)
        b = f.read(1)
        f.seek(grp.offset + grp.stride + 17)
        f.write(bytes([b[0] ^ 0x40]))
    grp.read(0)
    with pytest.raises(ff.FormatError, match="checksum"):
        grp.read(1)
    idx = json.load(open(os.path.join(dst, "index.json")))
    idx["version"] = 1
    json.dump(idx, open(os.path.join(dst, "index.json"), "w"))
    with pytest.raises(ff.FormatError, match="unsupported format"):
        ff.open_fp8_group(dst, 0)


@pytest.mark.gpu
def test_decode_runs_on_converted_records(tmp_path):
    """The one-launch decode step on records read back from a converted directory."""
    import torch

    hip.lib()  # raises if the library is missing: no fallback
    src, dst = str(tmp_path / "src"), str(tmp_path / "dst")
    hidden, inter, E, k, T = 256, 128, 16, 4, 3
    recs, _, parts = bf16_group(hidden, inter, E, 31)
    write_model(src, [(0, "bf16", recs, parts)])
    ff.convert_model(src, dst)
    grp = ff.open_fp8_group(dst, 0)
    frecs = [grp.read(e) for e in range(E)]
    geo = oracle.record_geometry(hidden, inter)
    rng = np.random.default_rng(8)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    xb = oracle.bf16_from_f32(rng.standard_normal((T, hidden)).astype(np.float32))
    want_ids, want_w, want = oracle.moe_decode(logits, oracle.bf16_to_f32(xb), frecs, k, geo)
    buf = torch.from_numpy(np.stack(frecs)).cuda()
    addrs = torch.tensor([buf.data_ptr() + e * grp.stride for e in range(E)], dtype=torch.int64, device="cuda")
    ws = torch.zeros(hip.moe_decode_fp8_workspace_size(T, E, k, grp.geo), dtype=torch.uint8, device="cuda")
    ids = torch.empty((T, k), dtype=torch.int32, device="cuda")
    w = torch.empty((T, k), dtype=torch.float32, device="cuda")
    out = torch.empty((T, hidden), dtype=torch.float32, device="cuda")
    xd = torch.from_numpy(xb.view(np.int16)).cuda().view(torch.bfloat16)
    hip.moe_decode_fp8(torch.from_numpy(logits).cuda(), xd, addrs, k, grp.geo, ids, w, out, ws)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(ids.cpu().numpy(), want_ids)
    got = out.cpu().numpy()
    assert np.abs(got - want).max() <= 1e-5 * max(1.0, np.abs(want).max()), np.abs(got - want).max()

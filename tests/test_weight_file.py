"""The on-disk kernel-order weight file (lq_wfile_* / ling_compile), on the CPU: a synthetic sharded safetensors
checkpoint (one shard written by the safetensors library, one by hand) is compiled, and every blob must equal
the oracle's restatement of the reference's retile_* (src/core/stream_gemm.cu:705-780) byte for byte; the code
table must be the checkpoint's distinct scale bytes in ascending order; side tables must hold the checkpoint's
scales as FP32. Corruptions and malformed checkpoints must fail with the library's error, never load."""
import json
import os
import struct

import numpy as np
import pytest
import torch

import oracle as O

L = pytest.importorskip("ling_gemm")
import ling_compile as LC  # noqa: E402


def write_safetensors(path, tensors, metadata=None):
    """Minimal writer of the safetensors format: u64 header length, JSON header, packed data."""
    header, blobs, off = {}, [], 0
    if metadata:
        header["__metadata__"] = metadata
    for name, (dtype, shape, data) in tensors.items():
        b = np.ascontiguousarray(data).tobytes()
        header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [off, off + len(b)]}
        blobs.append(b)
        off += len(b)
    h = json.dumps(header).encode()
    h += b" " * (-len(h) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)


def _u8(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.uint8))


def make_checkpoint(d):
    rng = np.random.default_rng(7)
    W = {}
    # NVFP4, few distinct scales -> coded
    v1, s1, g1, _ = O.quant_nvfp4(O.normal_bf16(1, 0.02, (64, 512)))
    # NVFP4, > 64 distinct scales -> raw tiled
    v2 = rng.integers(0, 256, (32, 1024), dtype=np.uint8)
    s2 = (np.arange(32 * 128, dtype=np.int64) % 120 + 1).astype(np.uint8).reshape(32, 128)
    rng.shuffle(s2.reshape(-1))
    f8a = rng.integers(0, 256, (48, 256), dtype=np.uint8)
    f8b = rng.integers(0, 256, (32, 384), dtype=np.uint8)
    sb = (rng.random(32) + 0.5).astype(np.float32)
    f8c = rng.integers(0, 256, (256, 384), dtype=np.uint8)
    sc = (rng.random((2, 3)) + 0.25).astype(np.float32)
    norm = rng.integers(0, 65536, 512, dtype=np.uint16)
    W.update(v1=v1, s1=s1, g1=g1, v2=v2, s2=s2, f8a=f8a, f8b=f8b, sb=sb, f8c=f8c, sc=sc, norm=norm)

    import safetensors.torch as st
    shard1 = {
        "model.layers.0.mlp.gate_proj.weight": _u8(v1),
        "model.layers.0.mlp.gate_proj.weight_scale": _u8(s1).view(torch.float8_e4m3fn),
        "model.layers.0.mlp.gate_proj.weight_scale_2": torch.tensor(g1, dtype=torch.float32),
        "model.layers.0.mlp.gate_proj.input_scale": torch.tensor(0.125, dtype=torch.float32),
        "model.layers.0.mlp.up_proj.weight": _u8(f8a).view(torch.float8_e4m3fn),
        "model.layers.0.mlp.up_proj.weight_scale": torch.tensor([0.5], dtype=torch.bfloat16),
        "model.layers.0.mlp.up_proj.input_scale": torch.tensor(2.0, dtype=torch.float32),
        "model.norm.weight": torch.from_numpy(norm.view(np.int16)).view(torch.bfloat16),
    }
    st.save_file(shard1, os.path.join(d, "model-00001-of-00002.safetensors"), metadata={"format": "pt"})
    shard2 = {
        "model.layers.1.mlp.down_proj.weight": ("U8", v2.shape, v2),
        "model.layers.1.mlp.down_proj.weight_scale": ("F8_E4M3", s2.shape, s2),
        "model.layers.1.mlp.down_proj.weight_scale_2": ("F32", [1], np.float32([0.75])),
        "model.layers.1.mlp.gate_proj.weight": ("F8_E4M3", f8b.shape, f8b),
        "model.layers.1.mlp.gate_proj.weight_scale": ("F32", [32, 1], sb),
        "model.layers.1.mlp.up_proj.weight": ("F8_E4M3", f8c.shape, f8c),
        "model.layers.1.mlp.up_proj.weight_scale_inv": ("F32", [2, 3], sc),
    }
    write_safetensors(os.path.join(d, "model-00002-of-00002.safetensors"), shard2, {"format": "pt"})
    names = {**{k: "model-00001-of-00002.safetensors" for k in shard1},
             **{k: "model-00002-of-00002.safetensors" for k in shard2}}
    with open(os.path.join(d, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {"total_size": 0}, "weight_map": names}, f)
    return W


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    d = str(tmp_path_factory.mktemp("ckpt"))
    return d, make_checkpoint(d)


@pytest.fixture(scope="module")
def compiled(ckpt, tmp_path_factory):
    d, W = ckpt
    out = str(tmp_path_factory.mktemp("out") / "model.lqw")
    n = LC.compile_checkpoint(d, out, passthrough=True)
    assert n == 6
    return out, W


def test_host_retile_matches_oracle():
    rng = np.random.default_rng(3)
    # 2048 x 8192 FP8 = 8192 blocks: the host retile splits it over several threads
    for N, K in [(16, 128), (48, 384), (2048, 8192)]:
        q = rng.integers(0, 256, (N, K), dtype=np.uint8)
        assert np.array_equal(L.host_retile_fp8(q), O.retile_fp8(q))
    for N, K in [(16, 128), (80, 1024), (1024, 8192)]:
        v = rng.integers(0, 256, (N, K // 2), dtype=np.uint8)
        s = rng.integers(0, 40, (N, K // 16), dtype=np.uint8)
        assert np.array_equal(L.host_retile_nvfp4(v, s), O.retile_nvfp4(v, s))
        ok, _, code_of = O.scale_code_table(s)
        assert ok
        blob, raw = L.host_retile_nvfp4_coded(v, s, code_of)
        blob_o, raw_o = O.retile_nvfp4_coded(v, s, code_of)
        assert np.array_equal(blob, blob_o) and np.array_equal(raw, raw_o)


def test_host_retile_rejects_untileable_shapes():
    with pytest.raises(L.LingGemmError, match="N % 16"):
        L.host_retile_fp8(np.zeros((24, 128), np.uint8))
    with pytest.raises(L.LingGemmError, match="K % 128"):
        L.host_retile_nvfp4(np.zeros((16, 40), np.uint8), np.zeros((16, 5), np.uint8))


def test_compiled_entries_match_oracle(compiled):
    out, W = compiled
    with LC.WeightFile(out) as f:
        assert sorted(f.names()) == sorted([
            "model.layers.0.mlp.gate_proj", "model.layers.0.mlp.up_proj", "model.layers.1.mlp.down_proj",
            "model.layers.1.mlp.gate_proj", "model.layers.1.mlp.up_proj", "model.norm.weight"])
        for i in range(len(f)):
            f.verify(i)

        e = f.entry("model.layers.0.mlp.gate_proj")
        assert (e.kind, e.N, e.K) == (L.WENTRY_NVFP4_CODED, 64, 512)
        assert e.weight_scale == np.float32(W["g1"]) and e.input_scale == 0.125
        ok, _, code_of = O.scale_code_table(W["s1"])
        assert ok
        blob_o, raw_o = O.retile_nvfp4_coded(W["v1"], W["s1"], code_of)
        assert np.array_equal(e.blob, blob_o) and np.array_equal(e.aux, raw_o)
        distinct = np.unique(W["s1"])  # the code table: distinct scale bytes, ascending, zero-padded
        assert np.array_equal(e.table[:distinct.size], distinct) and not e.table[distinct.size:].any()

        e = f.entry("model.layers.1.mlp.down_proj")
        assert (e.kind, e.N, e.K, e.weight_scale, e.input_scale) == (L.WENTRY_NVFP4, 32, 2048, 0.75, None)
        assert np.array_equal(e.blob, O.retile_nvfp4(W["v2"], W["s2"])) and e.aux is None and e.table is None

        e = f.entry("model.layers.0.mlp.up_proj")
        assert (e.kind, e.scale_kind, e.N, e.K, e.weight_scale, e.input_scale) == (
            L.WENTRY_FP8, L.WSCALE_TENSOR, 48, 256, 0.5, 2.0)
        assert np.array_equal(e.blob, O.retile_fp8(W["f8a"])) and e.aux is None

        e = f.entry("model.layers.1.mlp.gate_proj")
        assert (e.kind, e.scale_kind, e.N, e.K) == (L.WENTRY_FP8, L.WSCALE_CHANNEL, 32, 384)
        assert np.array_equal(e.blob, O.retile_fp8(W["f8b"]))
        assert np.array_equal(e.aux.view(np.float32), W["sb"])

        e = f.entry("model.layers.1.mlp.up_proj")
        assert (e.kind, e.scale_kind, e.N, e.K) == (L.WENTRY_FP8, L.WSCALE_BLOCK128, 256, 384)
        assert np.array_equal(e.blob, O.retile_fp8(W["f8c"]))
        assert np.array_equal(e.aux.view(np.float32).reshape(2, 3), W["sc"])

        e = f.entry("model.norm.weight")
        assert (e.kind, e.dtype, e.shape) == (L.WENTRY_RAW, "BF16", (512,))
        assert np.array_equal(e.blob.view(np.uint16), W["norm"])

        # sections start on 4096-byte boundaries of the file
        base = f.entry(0).blob.ctypes.data - (f.entry(0).blob.ctypes.data % 4096)
        for i in range(len(f)):
            for a in (f.entry(i).blob, f.entry(i).aux, f.entry(i).table):
                if a is not None:
                    assert (a.ctypes.data - base) % 4096 == 0


def test_compile_flags(ckpt, tmp_path):
    d, W = ckpt
    out = str(tmp_path / "raw.lqw")
    assert LC.compile_checkpoint(d, out, codes=False) == 5  # no pass-through: the norm is left out
    with LC.WeightFile(out) as f:
        e = f.entry("model.layers.0.mlp.gate_proj")
        assert e.kind == L.WENTRY_NVFP4 and np.array_equal(e.blob, O.retile_nvfp4(W["v1"], W["s1"]))
        with pytest.raises(KeyError):
            f.index("model.norm.weight")
    assert not os.path.exists(out + ".partial")


def test_compile_is_deterministic(ckpt, compiled, tmp_path):
    d, _ = ckpt
    out2 = str(tmp_path / "again.lqw")
    LC.compile_checkpoint(d, out2, passthrough=True)
    assert open(compiled[0], "rb").read() == open(out2, "rb").read()


def _corrupt_copy(src, dst, off, xor=0x40, truncate=None):
    b = bytearray(open(src, "rb").read())
    if truncate is not None:
        b = b[:truncate]
    else:
        b[off] ^= xor
    open(dst, "wb").write(bytes(b))


def test_corruption_is_detected(compiled, tmp_path):
    out, _ = compiled
    raw = open(out, "rb").read()
    # entry 0's blob offset: the record's u64 at byte 96 (header 64 bytes, records 192 bytes)
    blob_off = struct.unpack_from("<Q", raw, 64 + 96)[0]
    assert blob_off % 4096 == 0
    bad = str(tmp_path / "blob.lqw")
    _corrupt_copy(out, bad, blob_off + 5)
    with LC.WeightFile(bad) as f:
        f.verify(1)
        with pytest.raises(L.LingGemmError, match="blob hash mismatch"):
            f.verify(0)
    _corrupt_copy(out, bad, 64 + 20)  # inside entry 0
    with pytest.raises(L.LingGemmError, match="hash mismatch"):
        LC.WeightFile(bad)
    _corrupt_copy(out, bad, 0)
    with pytest.raises(L.LingGemmError, match="bad magic"):
        LC.WeightFile(bad)
    _corrupt_copy(out, bad, 0, truncate=len(raw) - 4096)
    with pytest.raises(L.LingGemmError, match="truncated"):
        LC.WeightFile(bad)
    with pytest.raises(L.LingGemmError, match="cannot open"):
        LC.WeightFile(str(tmp_path / "missing.lqw"))


def _single(d, tensors):
    os.makedirs(d, exist_ok=True)
    write_safetensors(os.path.join(d, "model.safetensors"), tensors)
    return d


def test_malformed_checkpoints_fail(tmp_path):
    out = str(tmp_path / "x.lqw")
    z = np.zeros
    cases = [
        ("N % 16", {"a.weight": ("F8_E4M3", [24, 128], z((24, 128), np.uint8)), "a.weight_scale": ("F32", [], z(1, np.float32))}),
        ("weight_scale_2", {"a.weight": ("U8", [16, 64], z((16, 64), np.uint8)),
                            "a.weight_scale": ("F8_E4M3", [16, 8], z((16, 8), np.uint8))}),
        ("\\[N\\]\\[K/16\\]", {"a.weight": ("U8", [16, 64], z((16, 64), np.uint8)),
                               "a.weight_scale": ("F8_E4M3", [16, 4], z((16, 4), np.uint8)),
                               "a.weight_scale_2": ("F32", [], z(1, np.float32))}),
        ("without weight_scale", {"a.weight": ("F8_E4M3", [16, 128], z((16, 128), np.uint8))}),
        ("per-channel", {"a.weight": ("F8_E4M3", [16, 128], z((16, 128), np.uint8)),
                         "a.weight_scale": ("F32", [8], z(8, np.float32))}),
        ("no quantized", {"norm.weight": ("BF16", [4], z(4, np.uint16))}),
    ]
    for i, (msg, t) in enumerate(cases):
        d = _single(str(tmp_path / f"c{i}"), t)
        with pytest.raises(L.LingGemmError, match=msg):
            LC.compile_checkpoint(d, out)
    # bytes that do not match shape and dtype
    d = str(tmp_path / "short")
    os.makedirs(d)
    write_safetensors(os.path.join(d, "model.safetensors"), {"a.weight": ("F8_E4M3", [16, 128], z((16, 64), np.uint8))})
    with pytest.raises(L.LingGemmError, match="do not match"):
        LC.compile_checkpoint(d, out)
    # a header that is not JSON, and an index naming a missing shard
    d = str(tmp_path / "badjson")
    os.makedirs(d)
    with open(os.path.join(d, "model.safetensors"), "wb") as f:
        f.write(struct.pack("<Q", 5) + b"{oops")
    with pytest.raises(L.LingGemmError, match="malformed JSON"):
        LC.compile_checkpoint(d, out)
    d = str(tmp_path / "noshard")
    os.makedirs(d)
    json.dump({"weight_map": {"a.weight": "gone.safetensors"}}, open(os.path.join(d, "model.safetensors.index.json"), "w"))
    with pytest.raises(L.LingGemmError, match="cannot open"):
        LC.compile_checkpoint(d, out)
    with pytest.raises(L.LingGemmError, match="no model.safetensors"):
        LC.compile_checkpoint(str(tmp_path / "empty_dir_does_not_exist"), out)
    assert not os.path.exists(out)


def test_escaped_names_and_metadata(tmp_path):
    d = str(tmp_path / "esc")
    q = np.arange(16 * 128, dtype=np.uint32).astype(np.uint8).reshape(16, 128)
    os.makedirs(d)
    # hand-written header: escaped characters in the name and a __metadata__ object
    hdr = ('{"__metadata__":{"format":"pt"},"a\\/b\\u00e9.weight":{"dtype":"F8_E4M3","shape":[16,128],'
           '"data_offsets":[0,2048]},"a\\/b\\u00e9.weight_scale":{"dtype":"F32","shape":[],'
           '"data_offsets":[2048,2052]}}').encode()
    with open(os.path.join(d, "model.safetensors"), "wb") as f:
        f.write(struct.pack("<Q", len(hdr)) + hdr + q.tobytes() + np.float32(3.0).tobytes())
    out = str(tmp_path / "e.lqw")
    LC.compile_checkpoint(d, out)
    with LC.WeightFile(out) as f:
        e = f.entry("a/bé")
        assert e.weight_scale == 3.0 and np.array_equal(e.blob, O.retile_fp8(q))


def test_cli(ckpt, tmp_path, capsys):
    d, _ = ckpt
    out = str(tmp_path / "cli.lqw")
    assert LC.main([d, out, "--list"]) == 0
    text = capsys.readouterr().out
    assert "5 entries" in text and "nvfp4-coded" in text and "block128" in text


def test_hostile_headers_fail(tmp_path):
    out = str(tmp_path / "h.lqw")
    # an element count that overflows 64 bits, and dimensions past the GEMM interface's int range
    for i, shape in enumerate([[1 << 40, 1 << 40, 1 << 40], [1 << 31, 128]]):
        d = str(tmp_path / f"h{i}")
        os.makedirs(d)
        hdr = json.dumps({"a.weight": {"dtype": "F8_E4M3", "shape": shape, "data_offsets": [0, 0]},
                          "a.weight_scale": {"dtype": "F32", "shape": [], "data_offsets": [0, 4]}}).encode()
        with open(os.path.join(d, "model.safetensors"), "wb") as f:
            f.write(struct.pack("<Q", len(hdr)) + hdr + b"\0" * 4)
        with pytest.raises(L.LingGemmError, match="too large|do not match"):
            LC.compile_checkpoint(d, out)
    # a NUL inside a tensor name
    d = str(tmp_path / "nul")
    os.makedirs(d)
    hdr = b'{"a\\u0000b.weight":{"dtype":"F8_E4M3","shape":[16,128],"data_offsets":[0,2048]}}'
    with open(os.path.join(d, "model.safetensors"), "wb") as f:
        f.write(struct.pack("<Q", len(hdr)) + hdr + b"\0" * 2048)
    with pytest.raises(L.LingGemmError, match="bad tensor name"):
        LC.compile_checkpoint(d, out)
    # a header length past the end of the file
    d = str(tmp_path / "len")
    os.makedirs(d)
    with open(os.path.join(d, "model.safetensors"), "wb") as f:
        f.write(struct.pack("<Q", 1 << 40) + b"{}")
    with pytest.raises(L.LingGemmError, match="bad header length"):
        LC.compile_checkpoint(d, out)


def test_compile_quantizes_high_precision_linears(tmp_path):
    """--quantize: BF16 / F32 linears become FP8 per-channel, FP8 block or NVFP4 entries equal to the library's
    host quantizers (pinned against the oracle in test_quantize.py) followed by the retile; embeddings, norms and
    untileable matrices are left to the passthrough."""
    d = str(tmp_path / "hp")
    wb = O.normal_bf16(41, 0.02, (64, 256))
    wf = O.normal_f32(42, 0.02, (32, 384))
    emb = O.normal_bf16(43, 0.02, (64, 256))
    odd = O.normal_bf16(44, 0.02, (24, 256))  # N % 16 != 0
    router = O.normal_bf16(45, 0.02, (32, 256))  # MoE router gates (N = #experts) stay as they are
    _single(d, {"m.q_proj.weight": ("BF16", wb.shape, wb), "m.o_proj.weight": ("F32", wf.shape, wf),
                "m.mlp.gate.weight": ("BF16", router.shape, router), "m.mlp.router.weight": ("BF16", router.shape, router),
                "m.mlp.gate_proj.weight": ("BF16", wb.shape, wb),
                "m.o_proj.input_scale": ("F32", [], np.float32([0.5])),
                "m.embed_tokens.weight": ("BF16", emb.shape, emb), "m.odd.weight": ("BF16", odd.shape, odd),
                "m.post_norm.weight": ("BF16", (256,), wb[0])})
    for mode in ("fp8", "fp8-block", "nvfp4"):
        out = str(tmp_path / f"{mode}.lqw")
        n = LC.compile_checkpoint(d, out, quantize=mode, passthrough=True)
        assert n == 8
        with LC.WeightFile(out) as f:
            assert {f.entry(i).name for i in range(len(f))} == {"m.q_proj", "m.o_proj", "m.embed_tokens.weight",
                                                                 "m.odd.weight", "m.post_norm.weight",
                                                                 "m.mlp.gate.weight", "m.mlp.router.weight",
                                                                 "m.mlp.gate_proj"}
            for name, src, dt in (("m.q_proj", wb, "BF16"), ("m.o_proj", wf, "F32"), ("m.mlp.gate_proj", wb, "BF16")):
                e = f.entry(name)
                f.verify(name)
                assert e.quantized and e.dtype == dt
                N, K = src.shape
                if mode == "nvfp4":
                    bf = src if dt == "BF16" else O.f32_to_bf16(src)
                    v, s, g, _ = L.quantize_nvfp4(bf)
                    assert np.float32(e.weight_scale) == np.float32(g)
                    if e.kind == L.WENTRY_NVFP4_CODED:
                        ok, table, code_of = L.scale_code_table(s)
                        blob, raw = O.retile_nvfp4_coded(v, s, code_of)
                        assert np.array_equal(e.blob, blob) and np.array_equal(e.aux, raw)
                    else:
                        assert np.array_equal(e.blob, O.retile_nvfp4(v, s))
                else:
                    q, s = (L.quantize_fp8_channel if mode == "fp8" else L.quantize_fp8_block128)(src)
                    assert e.kind == L.WENTRY_FP8
                    assert e.scale_kind == (L.WSCALE_CHANNEL if mode == "fp8" else L.WSCALE_BLOCK128)
                    assert np.array_equal(e.blob, O.retile_fp8(q))
                    assert np.array_equal(e.aux.view(np.float32), s.reshape(-1))
            assert f.entry("m.o_proj").input_scale == 0.5
            for raw in ("m.embed_tokens.weight", "m.odd.weight", "m.post_norm.weight", "m.mlp.gate.weight",
                        "m.mlp.router.weight"):
                assert f.entry(raw).kind == L.WENTRY_RAW
    with pytest.raises(L.LingGemmError, match="at most one"):
        L._check(L.lib.lq_wfile_compile(d.encode(), str(tmp_path / "x.lqw").encode(),
                                        L.WFILE_QUANT_FP8 | L.WFILE_QUANT_NVFP4, None))


def _rehash_meta(b: bytearray) -> None:
    """Recompute the entry-table hash after editing an entry, so that only the new bound checks can catch it."""
    strings_off, strings_bytes = struct.unpack_from("<QQ", b, 24)
    struct.pack_into("<Q", b, 56, _hash64(bytes(b[64:strings_off + strings_bytes])))


def _hash64(data: bytes) -> int:
    """FNV-1a over little-endian 64-bit words, the tail zero-padded, seeded with the byte count (the file's hash)."""
    h = (0xcbf29ce484222325 ^ len(data)) & 0xFFFFFFFFFFFFFFFF
    pad = data + b"\0" * (-len(data) % 8)
    for (w,) in struct.iter_unpack("<Q", pad):
        h ^= w
        h = (h * 0x100000001b3) & 0xFFFFFFFFFFFFFFFF
    return h


def test_hostile_entries_fail(compiled, tmp_path):
    """Entries that pass the hash but lie about their sizes or names: a name offset that wraps, a blob shorter than
    the tiled size of the entry's N and K, an aux table of the wrong size."""
    out, _ = compiled
    raw = bytearray(open(out, "rb").read())
    _rehash_meta(raw)
    assert bytes(raw) == open(out, "rb").read()  # the restated hash is the file's
    bad = str(tmp_path / "hostile.lqw")
    rec = 64  # entry 0
    cases = [
        (rec + 0, "<Q", 0xFFFFFFFFFFFFFFF0, "bad name"),          # name_off + name_len wraps
        (rec + 104, "<Q", 4096, "section sizes"),                  # blob_bytes smaller than tiled_bytes(N, K)
        (rec + 120, "<Q", 12, "section sizes|out of the file"),   # aux_bytes wrong for the kind
    ]
    for off, fmt, val, msg in cases:
        b = bytearray(raw)
        struct.pack_into(fmt, b, off, val)
        _rehash_meta(b)
        open(bad, "wb").write(bytes(b))
        with pytest.raises(L.LingGemmError, match=msg):
            LC.WeightFile(bad)

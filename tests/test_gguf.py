"""The native GGUF reader (inferno.jl_amd/csrc/gguf.hip) against files written
here from the format description (src/GGUF.jl:1-165 reads the same layout):
header, every key/value type (nested arrays included), tensor infos, the data
section at the next multiple of general.alignment, and the byte size of each
tensor by its block type.  Parsing needs no GPU; the upload test does.

The writer below is independent of the reader: it lays out bytes from the
field list and computes where the data section must start by itself.
"""
import struct
from pathlib import Path

import numpy as np
import pytest

from inferno_hip import synth

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
SCALAR_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f",
              BOOL: "<?", U64: "<Q", I64: "<q", F64: "<d"}


def enc_str(s: bytes) -> bytes:
    return struct.pack("<Q", len(s)) + s


def enc_value(t, v) -> bytes:
    if t == STR:
        return enc_str(v)
    if t == ARR:
        at, items = v
        return struct.pack("<IQ", at, len(items)) + b"".join(enc_value(at, x) for x in items)
    return struct.pack(SCALAR_FMT[t], v)


def gguf_bytes(kvs, tensors, alignment=None, version=3, magic=b"GGUF"):
    """kvs: [(key, type, value)]; tensors: [(name, dims, ggml_type, payload)].
    Returns (file bytes, data_offset, {name: offset})."""
    al = alignment or 32
    head = magic + struct.pack("<IQQ", version, len(tensors), len(kvs))
    for k, t, v in kvs:
        head += enc_str(k.encode()) + struct.pack("<I", t) + enc_value(t, v)
    offsets, data, off = {}, b"", 0
    for name, dims, gt, payload in tensors:
        off = -(-off // al) * al
        offsets[name] = off
        data = data.ljust(off, b"\0") + payload
        off += len(payload)
        head += enc_str(name.encode()) + struct.pack("<I", len(dims))
        head += b"".join(struct.pack("<Q", d) for d in dims) + struct.pack("<IQ", gt, offsets[name])
    data_offset = -(-len(head) // al) * al
    return head.ljust(data_offset, b"\0") + data, data_offset, offsets


def sample_tensors(rng):
    out = []
    for name, gt, inner, outer in (("blk.0.ffn_gate.weight", synth.Q4_K, 512, 3),
                                   ("blk.0.ffn_down.weight", synth.Q6_K, 2048, 2),
                                   ("blk.0.attn_v.weight", synth.Q5_K, 256, 4),
                                   ("output.weight", synth.Q8_0, 64, 5)):
        out.append((name, (inner, outer), gt, synth.weight(rng, gt, outer, inner).tobytes()))
    out.append(("output_norm.weight", (16,), 0, np.arange(16, dtype=np.float32).tobytes()))
    return out


ALL_KVS = [
    ("general.architecture", STR, b"qwen35"),
    ("u8", U8, 200), ("i8", I8, -7), ("u16", U16, 65000), ("i16", I16, -30000),
    ("u32", U32, 4000000000), ("i32", I32, -123456), ("f32", F32, 1.5), ("flag", BOOL, True),
    ("u64", U64, 2 ** 60), ("i64", I64, -2 ** 50), ("f64", F64, 2.25),
    ("tokenizer.ggml.tokens", ARR, (STR, [b"<s>", b"</s>", b"hello"])),
    ("ints", ARR, (I32, [1, -2, 3])),
    ("nested", ARR, (ARR, [(U8, [1, 2]), (U8, []), (U8, [3])])),
]


def open_file(tmp_path, blob, name="m.gguf"):
    from inferno_hip import GGUF
    p = tmp_path / name
    p.write_bytes(blob)
    return GGUF.read_gguf(p)


@pytest.mark.parametrize("alignment", [None, 64])
def test_reader_recovers_every_field(tmp_path, alignment):
    from inferno_hip import GGUF
    rng = synth.rng_for(0x6606)
    tensors = sample_tensors(rng)
    kvs = list(ALL_KVS)
    if alignment:
        kvs.append(("general.alignment", U32, alignment))
    blob, data_offset, offsets = gguf_bytes(kvs, tensors, alignment)
    with open_file(tmp_path, blob) as f:
        assert f.version == 3
        assert f.alignment == (alignment or 32)
        assert f.data_offset == data_offset
        assert sorted(f.tensors) == sorted(t[0] for t in tensors)
        for name, dims, gt, payload in tensors:
            info = f.tensors[name]
            assert info.dimensions == tuple(dims)
            assert info.type == gt
            assert info.offset == offsets[name]
            assert info.nbytes == len(payload)  # block size of the type, not 4 per element
            got = GGUF.get_tensor_raw_bytes(f, name)
            assert got.tobytes() == payload
        with pytest.raises(Exception, match="Tensor not found"):
            GGUF.get_tensor_raw_bytes(f, "missing.weight")


def test_header_ending_on_the_alignment_needs_no_padding(tmp_path):
    # grow a string until the tensor infos end exactly on a multiple of 32
    # (src/GGUF.jl:153-157 skips nothing then)
    tensors = [("w", (32,), 0, np.ones(32, np.float32).tobytes())]
    for pad in range(32):
        kvs = [("general.name", STR, b"x" * pad)]
        blob, data_offset, _ = gguf_bytes(kvs, tensors)
        head_len = 4 + 4 + 8 + 8 + (8 + 12 + 4 + 8 + pad) + (8 + 1 + 4 + 8 + 4 + 8)
        if head_len % 32 == 0:
            assert data_offset == head_len
            with open_file(tmp_path, blob) as f:
                assert f.data_offset == head_len
            return
    pytest.fail("no padding length put the header on the boundary")


def test_version_2_is_read(tmp_path):
    blob, data_offset, _ = gguf_bytes(ALL_KVS[:3], sample_tensors(synth.rng_for(1))[:1], version=2)
    with open_file(tmp_path, blob) as f:
        assert f.version == 2 and f.data_offset == data_offset


def _expect_error(tmp_path, blob, match):
    from inferno_hip import GGUF
    p = tmp_path / "bad.gguf"
    p.write_bytes(blob)
    with pytest.raises(Exception, match=match):
        GGUF.read_gguf(p)


def test_refuses_bad_files(tmp_path):
    rng = synth.rng_for(0x6607)
    tensors = sample_tensors(rng)
    good, data_offset, _ = gguf_bytes(ALL_KVS, tensors)
    _expect_error(tmp_path, b"GGUX" + good[4:], "magic")
    _expect_error(tmp_path, gguf_bytes(ALL_KVS, tensors, version=1)[0], "version")
    _expect_error(tmp_path, good[: data_offset - 40], "ends")             # inside the tensor infos
    _expect_error(tmp_path, good[:-1], "past the end")                    # last tensor cut short
    huge = b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 2 ** 21)
    _expect_error(tmp_path, huge + b"\0" * 64, "1 MiB")                   # src/GGUF.jl:76-78
    rank5 = gguf_bytes([], [("w", (1, 1, 1, 1, 32), 0, np.ones(32, np.float32).tobytes())])[0]
    _expect_error(tmp_path, rank5, "rank")
    dup = gguf_bytes([], [("w", (32,), 0, b"\0" * 128), ("w", (32,), 0, b"\0" * 128)])[0]
    _expect_error(tmp_path, dup, "duplicate")
    odd = gguf_bytes([], [("q", (100, 2), synth.Q4_K, b"\0" * 288)])[0]
    _expect_error(tmp_path, odd, "multiple of the block size")


@pytest.mark.gpu
def test_uploaded_tensors_feed_the_gemv(tmp_path):
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import oracle
    from inferno_hip import GGUF, _lib
    from inferno_hip.device import _stream
    rng = synth.rng_for(0x6608)
    specs = (("blk.0.ffn_up.weight", synth.Q4_K, 1024, 37), ("blk.0.ffn_down.weight", synth.Q6_K, 2048, 19),
             ("output.weight", synth.Q8_0, 256, 11))
    tensors = [(n, (i, o), t, synth.weight(rng, t, o, i).tobytes()) for n, t, i, o in specs]
    blob, _, _ = gguf_bytes([("general.alignment", U32, 64)], tensors, 64)
    with open_file(tmp_path, blob) as f:
        for name, gt, inner, outer in specs:
            print(f"[case] GGUF upload {name} type {gt} {outer}x{inner}", flush=True)
            h = GGUF.upload(f, name)
            w = GGUF.get_tensor_raw_bytes(f, name)
            x = synth.activations(rng, inner)
            xd = torch.from_numpy(x).cuda()
            yd = torch.empty(outer, device="cuda")
            _lib.check(_lib.lib().ihip_gemv_dev(gt, GGUF.device_ptr(h), xd.data_ptr(), yd.data_ptr(),
                                                inner, outer, _stream(None)))
            torch.cuda.synchronize()
            ref = oracle.gemv_f64(gt, w, x, inner, outer)
            tol = oracle.tolerance(oracle.row_norms(gt, w, inner, outer), x)
            assert np.all(np.abs(yd.cpu().numpy().astype(np.float64) - ref) <= tol)
            _lib.check(_lib.lib().ihip_weight_release(h))


@pytest.mark.gpu
def test_grouped_tensors_feed_one_gemv(tmp_path):
    """wq, wk and wv (src/ModelCPU.jl:789-791) uploaded back to back, from
    the file and from host arrays: one GEMV over the group gives every
    member's outputs, bit-identical to each member's own GEMV; each member's
    blocks sit at ihip_weight_bytes of the rows before it; tensors of another
    type or row length, and unknown names, are refused."""
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import oracle
    from inferno_hip import GGUF, _lib
    from inferno_hip import device as D
    from inferno_hip._lib import IHIPArgumentError
    rng = synth.rng_for(0x6609)
    inner = 2048
    specs = (("blk.0.attn_q.weight", 2048), ("blk.0.attn_k.weight", 256), ("blk.0.attn_v.weight", 256))
    for gt in (synth.Q4_K, synth.Q6_K):
        tensors = [(n, (inner, o), gt, synth.weight(rng, gt, o, inner).tobytes()) for n, o in specs]
        tensors.append(("blk.0.ffn_up.weight", (1024, 64), gt, synth.weight(rng, gt, 64, 1024).tobytes()))
        other = synth.Q8_0 if gt != synth.Q8_0 else synth.Q4_K
        tensors.append(("blk.0.attn_o.weight", (inner, 32), other, synth.weight(rng, other, 32, inner).tobytes()))
        blob, _, _ = gguf_bytes([("general.alignment", U32, 32)], tensors, 32)
        x = synth.activations(rng, inner)
        xd = torch.from_numpy(x).cuda()
        names = [n for n, _ in specs]
        outers = [o for _, o in specs]
        with open_file(tmp_path, blob, f"g{gt}.gguf") as f:
            print(f"[case] GGUF group upload type {gt}: rows {outers} x {inner}", flush=True)
            h = GGUF.upload_group(f, names)
            ws = [GGUF.get_tensor_raw_bytes(f, n) for n in names]
            total = sum(outers)
            y = torch.empty(total, device="cuda")
            _lib.check(_lib.lib().ihip_gemv_dev(gt, GGUF.device_ptr(h), xd.data_ptr(), y.data_ptr(),
                                                inner, total, D._stream(None)))
            grp = D.WeightGroup(ws, gt, inner, outers)
            y2 = grp.gemv(xd)
            o = 0
            for i, (w, r) in enumerate(zip(ws, outers)):
                own = D.gemv(D.DeviceWeight(torch.from_numpy(w).cuda(), gt, inner, r), xd).cpu().numpy()
                got = y[o:o + r].cpu().numpy()
                ref = oracle.gemv_f64(gt, w, x, inner, r)
                tol = oracle.tolerance(oracle.row_norms(gt, w, inner, r), x)
                assert np.all(np.abs(got.astype(np.float64) - ref) <= tol), f"member {i}"
                assert np.array_equal(got.view(np.uint32), own.view(np.uint32)), f"member {i} (file group)"
                assert np.array_equal(y2[o:o + r].cpu().numpy().view(np.uint32), own.view(np.uint32))
                # the member's blocks inside the group
                assert _lib.lib().ihip_weight_bytes(gt, inner, o) == o * w.size // r
                torch.cuda.synchronize()
                assert torch.equal(torch.from_numpy(w).cuda(), _device_bytes(torch, grp.member_ptr(i), w.size))
                o += r
            grp.release()
            _lib.check(_lib.lib().ihip_weight_release(h))
            with pytest.raises(IHIPArgumentError, match="share one type"):
                GGUF.upload_group(f, names + ["blk.0.attn_o.weight"])
            with pytest.raises(IHIPArgumentError, match="share one type"):
                GGUF.upload_group(f, names + ["blk.0.ffn_up.weight"])
            with pytest.raises(IHIPArgumentError, match="not found"):
                GGUF.upload_group(f, names + ["blk.9.attn_q.weight"])


def _device_bytes(torch, ptr, n):
    """n bytes at a device address, copied into a fresh device tensor."""
    import ctypes as C
    out = torch.empty(n, dtype=torch.uint8, device="cuda")
    hip = C.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    assert hip.hipMemcpy(out.data_ptr(), ptr, n, 3) == 0  # device to device
    return out


def test_bench_writer_round_trips(tmp_path):
    """bench.py's GGUF writer (the file its registry-load leg times) is read
    back by the native reader: names, types, dimensions and bytes."""
    import sys
    root = Path(__file__).resolve().parents[1]
    if str(root) not in sys.path:
        sys.path.insert(0, str(root))
    import bench
    from inferno_hip import GGUF
    rng = synth.rng_for(0x66)
    tensors = [("blk.0.ffn_gate.weight", synth.Q4_K, (512, 3), synth.weight(rng, synth.Q4_K, 3, 512)),
               ("output.weight", synth.Q6_K, (256, 5), synth.weight(rng, synth.Q6_K, 5, 256)),
               ("q8", synth.Q8_0, (64, 7), synth.weight(rng, synth.Q8_0, 7, 64))]
    path = tmp_path / "bench.gguf"
    bench.write_gguf(str(path), tensors)
    with GGUF.read_gguf(path) as f:
        assert f.version == 3 and f.alignment == 32
        for name, t, dims, blob in tensors:
            info = f.tensors[name]
            assert (info.type, info.dimensions, info.nbytes) == (t, dims, blob.size)
            assert np.array_equal(GGUF.get_tensor_raw_bytes(f, name), blob)

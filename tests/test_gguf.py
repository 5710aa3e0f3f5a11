"""GGUF reader parity on the CPU: every fixture under tests/golden/gguf is
opened through the C-ABI (flh_gguf_*) and compared with what the reference's
own reader (fastllm::Gguf, src/model/gguf.cpp, compiled from its sources)
read from the same file, recorded in tests/golden/gguf_ref.json: alignment,
shard count, every tensor info, payload bytes (FNV-1a), find(), and every
metadata getter for every key.  Files the reference aborts on must give
FLH_ERR_FORMAT, files it reports missing FLH_ERR_IO.  Parsing touches no GPU.
"""
import json
import os

import numpy as np
import pytest

from gguf_writer import GgufFile
import gguf_writer as gw

HERE = os.path.dirname(os.path.abspath(__file__))
FIX = os.path.join(HERE, "golden", "gguf")
GOLD = json.load(open(os.path.join(HERE, "golden", "gguf_ref.json")))

# accepted by the reference, rejected here on purpose: a payload past the end
# of the file (the reference reads outside its mapping) and an alignment that
# is not a power of two (the reference rounds with a bit mask, which needs one)
STRICTER = {"tensor_past_eof.gguf", "align_48.gguf"}


def fnv1a(b: np.ndarray) -> int:
    h = 1469598103934665603
    for v in b.tobytes():
        h = ((h ^ v) * 1099511628211) & 0xFFFFFFFFFFFFFFFF
    return h


def raw(s: str) -> bytes:
    """A string from the golden record (bytes escaped one by one) as bytes."""
    return s.encode("latin-1")


def mine(s: str) -> bytes:
    return s.encode("utf-8", "surrogateescape")


@pytest.mark.parametrize("name", sorted(GOLD["files"]))
def test_reader_matches_reference(flh, name):
    want = GOLD["files"][name]
    path = os.path.join(FIX, name)
    if want["result"] == "signal" or name in STRICTER:
        with pytest.raises(flh.FlhError) as e:
            flh.Gguf(path)
        assert e.value.code == flh.ERR_FORMAT, e.value
        return
    if want["result"] == "false":
        with pytest.raises(flh.FlhError) as e:
            flh.Gguf(path)
        assert e.value.code == flh.ERR_IO, e.value
        return
    assert want["result"] == "ok"
    with flh.Gguf(path) as g:
        assert g.alignment() == want["alignment"]
        assert g.n_shards() == want["n_shards"]
        ts = g.tensors()
        assert len(ts) == len(want["tensors"])
        for t, w in zip(ts, want["tensors"]):
            assert mine(t.name) == raw(w["name"])
            assert (t.type, t.n_dims, list(t.ne), t.offset, t.nbytes, t.shard) == \
                (w["type"], w["n_dims"], w["ne"], w["offset"], w["nbytes"], w["shard"]), t.name
            assert (-1 if t.fmt < 0 else t.fmt) == w["fmt"]
            assert flh.Gguf.type_name(t.type) == w["type_name"]
            assert fnv1a(g.data(t)) == int(w["fnv"]), t.name
            assert (g.find(t.name) is t) == w["find_is_self"]
        for k, w in want["kv"].items():
            assert g.has(k) == w["has"], k
            assert g.kv_i(k, -777) == w["i"], k
            assert g.kv_f(k, -777.5) == w["f"], k
            assert mine(g.kv_s(k, "<none>")) == raw(w["s"]), k
            sa = g.kv_sarr(k)
            if w["sarr"] is None:
                assert sa is None, k
            else:
                assert [mine(x) for x in sa] == [raw(x) for x in w["sarr"]], k


def test_reference_reader_test_file(flh):
    """The reference's own reader round trip (tests/test_quants.cpp:140-206):
    names, types, dims, payload sizes and bytes of the five tensors."""
    with flh.Gguf(os.path.join(FIX, "basic.gguf")) as g:
        assert g.alignment() == 32 and len(g.tensors()) == 5
        blob = open(os.path.join(FIX, "basic.gguf"), "rb").read()
        spec = [("t.q8", 8, 64, 3, 34 * 2 * 3), ("t.q50", 6, 64, 2, 22 * 2 * 2),
                ("t.q4k", 12, 256, 2, 144 * 2), ("t.q6k", 14, 256, 1, 210),
                ("t.f32", 0, 16, 4, 256)]
        hdr_end = len(blob) - sum(-(-n // 32) * 32 for *_, n in spec[:-1]) - spec[-1][4]
        for name, ty, ne0, ne1, nb in spec:
            t = g.find(name)
            assert t is not None and t.type == ty and t.ne[:2] == (ne0, ne1) and t.nbytes == nb
            assert g.data(t).tobytes() == blob[hdr_end + t.offset:hdr_end + t.offset + nb]


def test_split_model_metadata_and_offsets(flh):
    """Shard 1 names the model and holds no tensors; the tensors of shards 2
    and 3 are merged with per-shard data offsets (shard 3 aligned to 64)."""
    with flh.Gguf(os.path.join(FIX, "model-00001-of-00003.gguf")) as g:
        assert g.n_shards() == 3
        assert g.kv_s("general.architecture") == "deepseek2"
        assert g.kv_i("split.no", -1) == 0 and not g.has("only.in.two")
        assert [t.shard for t in g.tensors()] == [1, 1, 2, 2, 2]
        assert g.kv_i("split.tensors.count", 0) == len(g.tensors())
    with flh.Gguf(os.path.join(FIX, "model-00002-of-00003.gguf")) as g:
        assert g.kv_s("general.architecture") == "shard2" and g.kv_f("only.in.two", 0) == 0.5


def test_weight_binding_like_load_tensor(flh):
    """DecoderImpl::load_tensor (src/model/decoder.cpp:186-206): fmt, cols =
    ne0, rows = ne1, nexp = ne2 of 3-D stacks, estride = rows * row_bytes."""
    with flh.Gguf(os.path.join(FIX, "kv_types.gguf")) as g:
        w = g.weight("blk.0.ffn_gate_exps.weight")
        assert (w.fmt, w.cols, w.rows, w.nexp) == (flh.Fmt.Q4_K, 256, 4, 3)
        assert w.row_bytes == 144 and w.w_bytes == 576 and w.estride == 576
        t = g.find("blk.0.ffn_gate_exps.weight")
        assert w.host == t.address and w.tensor == t.index
        w = g.weight("q5.odd")
        assert (w.fmt, w.rows, w.cols, w.nexp, w.estride) == (flh.Fmt.Q5_0, 5, 96, 1, 0)
        with pytest.raises(flh.FlhError) as e:
            g.weight("f16.3d")
        assert e.value.code == flh.ERR_UNSUPPORTED
        with pytest.raises(flh.FlhError) as e:
            g.weight("no.such.tensor")
        assert e.value.code == flh.ERR_ARG


def test_fmt_of_and_type_names(flh):
    """Gguf::fmt_of / type_name (src/model/gguf.cpp:82-109)."""
    want = {0: flh.Fmt.F32, 8: flh.Fmt.Q8_0, 6: flh.Fmt.Q5_0, 12: flh.Fmt.Q4_K,
            14: flh.Fmt.Q6_K, 16: flh.Fmt.IQ2_XXS, 18: flh.Fmt.IQ3_XXS}
    for t in range(40):
        assert flh.Gguf.fmt_of(t) == want.get(t)
    assert flh.Gguf.type_name(1) == "F16" and flh.Gguf.type_name(2) == "type2"


def test_missing_file_and_truncations(flh, tmp_path):
    with pytest.raises(flh.FlhError) as e:
        flh.Gguf(str(tmp_path / "nope.gguf"))
    assert e.value.code == flh.ERR_IO
    g = GgufFile(3)
    g.add_kv("tokenizer.ggml.tokens", gw.ARR, (gw.STR, ["a", "bb", "ccc"] * 50))
    g.add_tensor("w", gw.GGML_Q8_0, (64, 4), np.zeros(34 * 8, np.uint8))
    blob = g.to_bytes()
    hdr, _ = g.header_and_offsets()
    # every cut inside the header is FLH_ERR_FORMAT, never a crash
    for cut in list(range(0, 64)) + list(range(64, len(hdr), 7)):
        p = tmp_path / "cut.gguf"
        p.write_bytes(blob[:cut])
        with pytest.raises(flh.FlhError) as e:
            flh.Gguf(str(p))
        assert e.value.code == flh.ERR_FORMAT, cut
    # a cut inside the payload leaves the tensor past the end of the file
    p = tmp_path / "cut.gguf"
    p.write_bytes(blob[:-1])
    with pytest.raises(flh.FlhError):
        flh.Gguf(str(p))
    p.write_bytes(blob)
    with flh.Gguf(str(p)) as gg:
        assert gg.kv_sarr("tokenizer.ggml.tokens") == ["a", "bb", "ccc"] * 50


def test_unsized_array_element_is_rejected(flh, tmp_path):
    import struct
    b = (struct.pack("<IIQQ", 0x46554747, 3, 0, 1) + gw.gstr("k")
         + struct.pack("<IIQ", gw.ARR, 13, 2) + b"\0" * 16)
    p = tmp_path / "arr.gguf"
    p.write_bytes(b)
    with pytest.raises(flh.FlhError) as e:
        flh.Gguf(str(p))
    assert e.value.code == flh.ERR_FORMAT


def test_upload_needs_init(flh):
    """Nothing before flh_gguf_upload* touches the GPU; the upload itself
    refuses to run before flh_init (checked without a device)."""
    if getattr(flh, "_initialised", False):
        pytest.skip("device already initialised in this process")
    with flh.Gguf(os.path.join(FIX, "basic.gguf")) as g:
        t = g.find("t.q8")
        rc = flh.lib().flh_gguf_upload(g.handle, t.index, 4096, t.nbytes, None)
        assert rc == flh.ERR_STATE


@pytest.mark.parametrize("dims,why", [((256, 1 << 32, 1 << 32, 1), "dims whose product wraps 64 bits"),
                                      ((256, 1 << 62, 4), "byte count past 2^64"),
                                      ((300, 4), "row not a whole number of superblocks"),
                                      ((256 << 32, 1), "row wider than 2^32 - 1 elements")])
def test_impossible_sizes_are_rejected(flh, tmp_path, dims, why):
    """A header whose size arithmetic would wrap (and so slip past the
    end-of-file check) or whose rows cannot be a Q4_K row is FLH_ERR_FORMAT
    (the reference reader, src/model/gguf.cpp:248-256, multiplies unchecked)."""
    g = GgufFile(3)
    g.add_tensor("w", gw.GGML_Q4_K, dims, np.zeros(144, np.uint8))
    p = tmp_path / "big.gguf"
    g.write(str(p))
    with pytest.raises(flh.FlhError) as e:
        flh.Gguf(str(p))
    assert e.value.code == flh.ERR_FORMAT, why


def test_mutated_files_never_crash(flh, tmp_path):
    """Seeded byte mutations of every fixture (bytes flipped, 4- and 8-byte
    fields overwritten with boundary values, bytes cut or inserted in the
    header region): each file either opens, and every tensor info, lookup and
    metadata getter then works, or is rejected with an error code; the
    walk runs in a child process so that a crash fails the test instead of
    ending the session."""
    import random
    import struct
    import subprocess
    import sys
    rnd = random.Random(2026)
    blobs = [open(os.path.join(FIX, f), "rb").read() for f in sorted(os.listdir(FIX)) if f.endswith(".gguf")]
    blobs = [b for b in blobs if len(b) > 24]
    vals = [0, 1, 0x7F, 0x80, 0xFF, 0x7FFFFFFF, 0x80000000, 0xFFFFFFFF, 1 << 32, 1 << 40, (1 << 64) - 1]
    paths = []
    for i in range(400):
        b = bytearray(rnd.choice(blobs))
        for _ in range(rnd.randint(1, 6)):
            hdr = min(len(b), 4096)
            if hdr == 0:
                break
            pos, r = rnd.randrange(hdr), rnd.random()
            if r < 0.4:
                b[pos] = rnd.randrange(256)
            elif r < 0.7 and pos + 8 <= len(b):
                b[pos:pos + 8] = struct.pack("<Q", rnd.choice(vals))
            elif r < 0.85 and pos + 4 <= len(b):
                b[pos:pos + 4] = struct.pack("<I", rnd.choice(vals) & 0xFFFFFFFF)
            elif r < 0.93:
                del b[pos:pos + rnd.randint(1, 16)]
            else:
                b[pos:pos] = bytes(rnd.randrange(256) for _ in range(rnd.randint(1, 16)))
        p = tmp_path / f"m{i}.gguf"
        p.write_bytes(bytes(b))
        paths.append(str(p))
    code = r'''
import sys
sys.path.insert(0, sys.argv[1])
import importlib
flh = importlib.import_module("fast-llm_amd")
n = 0
for p in sys.argv[2:]:
    try:
        g = flh.Gguf(p)
    except flh.FlhError:
        continue
    n += 1
    with g:
        g.alignment()
        g.n_shards()
        for t in g.tensors():
            g.find(t.name)
            g.data(t)
            try:
                g.weight(t.name)
            except flh.FlhError:
                pass
        for k in ("general.architecture", "tokenizer.ggml.tokens", "general.alignment", "split.count"):
            g.has(k)
            g.kv_i(k, 0)
            g.kv_f(k, 0.0)
            g.kv_s(k, "")
            g.kv_sarr(k)
print("opened", n)
'''
    root = os.path.dirname(HERE)
    r = subprocess.run([sys.executable, "-c", code, root] + paths, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    assert r.stdout.startswith("opened")

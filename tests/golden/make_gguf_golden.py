"""Write the GGUF reader fixtures and record what the reference reads from them.

Runs ONLY in the build container, where /root/reference exists:
  make -C oracle ref && python tests/golden/make_gguf_golden.py
Writes small synthetic GGUF files under tests/golden/gguf/ with this repo's
own writer (tests/gguf_writer.py), then opens each one with the reference's
reader (fastllm::Gguf, src/model/gguf.cpp, compiled from its sources into
oracle/_ref/libflref_gguf.so by oracle/Makefile) in a child process, and
stores the result in tests/golden/gguf_ref.json: every tensor info with an
FNV-1a hash of its payload, the metadata getters for every key, or the way
open() ended (returned false, or the process died of SIGABRT / SIGSEGV).
The first fixture follows the reference's own reader test
(tests/test_quants.cpp:140-206).
"""
import ctypes
import json
import os
import struct
import subprocess
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
TESTS = os.path.dirname(HERE)
ROOT = os.path.dirname(TESTS)
sys.path.insert(0, TESTS)
import gguf_writer as gw  # noqa: E402
from gguf_writer import GgufFile  # noqa: E402

OUT = os.path.join(HERE, "gguf")
REF_SO = os.path.join(ROOT, "oracle", "_ref", "libflref_gguf.so")


def sane_blocks(ggml_type, ne, rng):
    """Random payload with small finite fp16 scales where a format has them."""
    n = gw.payload_bytes(ggml_type, ne)
    w = rng.integers(0, 256, size=n, dtype=np.uint8)
    if ggml_type in (gw.GGML_F32,):
        return rng.standard_normal(n // 4).astype(np.float32).view(np.uint8)
    if ggml_type == gw.GGML_F16:
        return rng.standard_normal(n // 2).astype(np.float16).view(np.uint8)
    bb = gw.GGML_BLOCK[ggml_type][1]
    blocks = w.reshape(-1, bb)
    half = lambda: (0x2000 | (rng.integers(0, 1 << 16, blocks.shape[0]) & 0x0BFF)).astype(np.uint16)
    if ggml_type == gw.GGML_Q6_K:
        blocks[:, 208:210] = half().view(np.uint8).reshape(-1, 2)
    elif ggml_type in (gw.GGML_Q8_0, gw.GGML_Q5_0, gw.GGML_Q4_K):
        blocks[:, 0:2] = half().view(np.uint8).reshape(-1, 2)
        if ggml_type == gw.GGML_Q4_K:
            blocks[:, 2:4] = half().view(np.uint8).reshape(-1, 2)
    return w


def fixtures(rng):
    """name -> bytes of every fixture file."""
    F = {}

    # 1. the reference reader test's file: five 2-D tensors, alignment 32
    g = GgufFile(3, alignment=32)
    for name, t, ne0, ne1 in [("t.q8", gw.GGML_Q8_0, 64, 3), ("t.q50", gw.GGML_Q5_0, 64, 2),
                              ("t.q4k", gw.GGML_Q4_K, 256, 2), ("t.q6k", gw.GGML_Q6_K, 256, 1),
                              ("t.f32", gw.GGML_F32, 16, 4)]:
        g.add_tensor(name, t, (ne0, ne1), sane_blocks(t, (ne0, ne1), rng))
    F["basic.gguf"] = g.to_bytes()

    # 2. every KV value type, arrays, nested arrays, repeated keys, v2,
    #    alignment 64 given as u64, and tensors of 1-4 dims / unsized types
    g = GgufFile(2)
    g.add_kv("general.architecture", gw.STR, "llama")
    g.add_kv("k.u8", gw.U8, 250).add_kv("k.i8", gw.I8, -7).add_kv("k.u16", gw.U16, 65000)
    g.add_kv("k.i16", gw.I16, -30000).add_kv("k.u32", gw.U32, 4000000000)
    g.add_kv("k.i32", gw.I32, -2000000000).add_kv("k.u64", gw.U64, (1 << 63) + 5)
    g.add_kv("k.i64", gw.I64, -(1 << 62)).add_kv("k.f32", gw.F32, 1.0e-6)
    g.add_kv("k.f64", gw.F64, -2.75).add_kv("k.bool1", gw.BOOL, 1).add_kv("k.bool0", gw.BOOL, 0)
    g.add_kv("k.bool7", gw.BOOL, 7)
    g.add_kv("k.str", gw.STR, "héllo 世界")
    g.add_kv("k.str_nul", gw.STR, b"a\0b")
    g.add_kv("k.str_empty", gw.STR, "")
    g.add_kv("tokenizer.ggml.tokens", gw.ARR, (gw.STR, ["<s>", "", "Ġthe", "a\nb", "ÿ"]))
    g.add_kv("tokenizer.ggml.scores", gw.ARR, (gw.F32, [0.0, -1.5, 2.25]))
    g.add_kv("k.arr_u16", gw.ARR, (gw.U16, [1, 2, 3]))
    g.add_kv("k.arr_empty", gw.ARR, (gw.I64, []))
    g.add_kv("k.arr_nested", gw.ARR, (gw.ARR, [(gw.STR, ["x", "yy"]), (gw.U8, [1, 2, 3]),
                                               (gw.ARR, [(gw.F64, [1.0])])]))
    g.add_kv("k.arr_str_empty", gw.ARR, (gw.STR, []))
    g.add_kv("k.dup", gw.I32, 1).add_kv("k.dup", gw.I32, 2)
    g.add_kv("k.dup_f", gw.F32, 1.5).add_kv("k.dup_f", gw.U8, 3)
    g.add_kv("k.dup_sarr", gw.ARR, (gw.STR, ["p", "q"])).add_kv("k.dup_sarr", gw.ARR, (gw.STR, ["r"]))
    g.add_kv("general.alignment", gw.U64, 64)
    g.add_kv("k.after_align", gw.STR, "tail")
    for name, t, dims in [("blk.0.ffn_gate_exps.weight", gw.GGML_Q4_K, (256, 4, 3)),
                          ("blk.0.attn_norm.weight", gw.GGML_F32, (32,)),
                          ("f16.3d", gw.GGML_F16, (8, 3, 2)),
                          ("q8.4d", gw.GGML_Q8_0, (64, 2, 2, 2)),
                          ("q6.wide", gw.GGML_Q6_K, (512, 3))]:
        g.add_tensor(name, t, dims, sane_blocks(t, dims, rng))
    g.add_tensor("q4_0.unsized", 2, (64, 2), rng.integers(0, 256, 72, dtype=np.uint8))
    g.add_tensor("iq2.xxs", gw.GGML_IQ2_XXS, (256, 2), rng.integers(0, 256, 132, dtype=np.uint8))
    g.add_tensor("dup.name", gw.GGML_F32, (4,), np.arange(4, dtype=np.float32))
    g.add_tensor("dup.name", gw.GGML_F32, (4,), np.arange(4, 8, dtype=np.float32))
    g.add_tensor("q5.odd", gw.GGML_Q5_0, (96, 5), sane_blocks(gw.GGML_Q5_0, (96, 5), rng))
    F["kv_types.gguf"] = g.to_bytes()

    # 3. no KV, no tensors
    F["empty.gguf"] = GgufFile(3).to_bytes()

    # 4. a split model: shard 1 holds only metadata, shards 2 and 3 the
    #    tensors; shard 3 has its own alignment; each shard has split.no
    def shard(no, kvs, tensors, align=None):
        g = GgufFile(3, alignment=align)
        g.add_kv("split.no", gw.U16, no).add_kv("split.count", gw.U16, 3)
        for k, t, v in kvs:
            g.add_kv(k, t, v)
        for name, t, dims in tensors:
            g.add_tensor(name, t, dims, sane_blocks(t, dims, rng))
        return g.to_bytes()
    t2 = [("s.q4k", gw.GGML_Q4_K, (512, 3)), ("s.q8", gw.GGML_Q8_0, (128, 2))]
    t3 = [("s.q6k", gw.GGML_Q6_K, (256, 2)), ("s.f32", gw.GGML_F32, (7, 3)),
          ("s.q50", gw.GGML_Q5_0, (32, 1))]
    F["model-00001-of-00003.gguf"] = shard(0, [("general.architecture", gw.STR, "deepseek2"),
                                                ("split.tensors.count", gw.I32, 5),
                                                ("deepseek2.block_count", gw.U32, 27)], [])
    F["model-00002-of-00003.gguf"] = shard(1, [("general.architecture", gw.STR, "shard2"),
                                                ("only.in.two", gw.F32, 0.5)], t2)
    F["model-00003-of-00003.gguf"] = shard(2, [], t3, align=64)
    # a single-shard "split" name is an ordinary file
    F["one-00001-of-00001.gguf"] = F["basic.gguf"]
    # a name that looks split but whose digits do not fit the pattern
    F["model-1-of-3.gguf"] = F["empty.gguf"]
    # shard 2 missing
    F["miss-00001-of-00002.gguf"] = shard(0, [], [("m.q8", gw.GGML_Q8_0, (32, 1))])
    # split.tensors.count disagrees with the shards
    F["bad-00001-of-00002.gguf"] = shard(0, [("split.tensors.count", gw.U64, 3)],
                                         [("b.q8", gw.GGML_Q8_0, (32, 1))])
    F["bad-00002-of-00002.gguf"] = shard(1, [], [("b.f32", gw.GGML_F32, (8, 1))])

    # 5. malformed files: the reference aborts on each
    good = F["basic.gguf"]
    F["bad_magic.gguf"] = b"GGUG" + good[4:]
    F["bad_version1.gguf"] = good[:4] + (1).to_bytes(4, "little") + good[8:]
    F["bad_version4.gguf"] = good[:4] + (4).to_bytes(4, "little") + good[8:]
    F["trunc_header.gguf"] = good[:20]
    hdr, _ = GgufFile(3, alignment=32).header_and_offsets()
    F["trunc_kv.gguf"] = good[:len(hdr) - 3]
    F["bad_kv_type.gguf"] = (struct.pack("<IIQQ", 0x46554747, 3, 0, 1) + gw.gstr("k.bad")
                             + struct.pack("<I", 13) + b"\0" * 16)
    for nd in (0, 5):
        g = GgufFile(3)
        g.add_tensor("t", gw.GGML_F32, (4,) * max(nd, 1), np.zeros(4 ** max(nd, 1), np.float32))
        b = bytearray(g.to_bytes())
        pos = 24 + 8 + 1
        b[pos:pos + 4] = nd.to_bytes(4, "little")
        F[f"bad_ndims{nd}.gguf"] = bytes(b)
    # a string whose length runs past the end of the file
    g = GgufFile(3)
    g.add_kv("k", gw.STR, "abc")
    b = bytearray(g.to_bytes())
    b[24 + 8 + 1 + 4:24 + 8 + 1 + 4 + 8] = (1 << 40).to_bytes(8, "little")
    F["bad_strlen.gguf"] = bytes(b)

    # 6. inputs this reader rejects but the reference accepts
    g = GgufFile(3)
    g.add_tensor("past.eof", gw.GGML_Q8_0, (64, 4), sane_blocks(gw.GGML_Q8_0, (64, 4), rng))
    F["tensor_past_eof.gguf"] = g.to_bytes()[:-40]
    g = GgufFile(3, alignment=48)
    g.add_tensor("a", gw.GGML_F32, (8,), np.ones(8, np.float32))
    F["align_48.gguf"] = g.to_bytes()
    return F


def all_keys(files):
    keys = {"absent.key", "general.name", "split.tensors.count", "split.count", "split.no"}
    for b in files.values():
        p = 24
        try:
            n_kv = int.from_bytes(b[16:24], "little")
            if b[:4] != b"GGUF" or n_kv > 1000:
                continue
            for _ in range(n_kv):
                n = int.from_bytes(b[p:p + 8], "little")
                keys.add(b[p + 8:p + 8 + n].decode())
                p += 8 + n
                t = int.from_bytes(b[p:p + 4], "little")
                p += 4
                p += _skip(b, p, t)
        except Exception:
            continue
    return sorted(keys)


def _skip(b, p, t):
    sizes = {0: 1, 1: 1, 2: 2, 3: 2, 4: 4, 5: 4, 6: 4, 7: 1, 10: 8, 11: 8, 12: 8}
    if t == gw.STR:
        return 8 + int.from_bytes(b[p:p + 8], "little")
    if t == gw.ARR:
        et = int.from_bytes(b[p:p + 4], "little")
        n = int.from_bytes(b[p + 4:p + 12], "little")
        q = p + 12
        for _ in range(n):
            q += _skip(b, q, et) if et in (gw.STR, gw.ARR) else sizes[et]
        return q - p
    return sizes[t]


CHILD = r"""
import ctypes, sys
L = ctypes.CDLL(sys.argv[1])
L.ref_gguf_dump.restype = ctypes.c_long
L.ref_gguf_dump.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p, ctypes.c_size_t]
buf = ctypes.create_string_buffer(1 << 22)
n = L.ref_gguf_dump(sys.argv[2].encode(), sys.argv[3].encode(), buf, len(buf))
sys.stdout.write("FALSE" if n < 0 else buf.value.decode())
"""


def reference_read(path, keys):
    r = subprocess.run([sys.executable, "-c", CHILD, REF_SO, path, "\n".join(keys)],
                       capture_output=True, text=True, timeout=60)
    if r.returncode < 0:
        return {"result": "signal", "signal": -r.returncode, "stderr": r.stderr.strip()[-200:]}
    if r.returncode != 0:
        return {"result": "error", "stderr": r.stderr.strip()[-400:]}
    if r.stdout == "FALSE":
        return {"result": "false"}
    return {"result": "ok", **json.loads(r.stdout)}


def main():
    if not os.path.exists(REF_SO):
        sys.exit(f"{REF_SO} missing: run make -C oracle ref")
    rng = np.random.default_rng(20261201)
    files = fixtures(rng)
    os.makedirs(OUT, exist_ok=True)
    for name, b in files.items():
        with open(os.path.join(OUT, name), "wb") as f:
            f.write(b)
    keys = all_keys(files)
    # the fixtures opened by name (a split model is opened through one shard)
    opened = [n for n in files if not (n.startswith(("model-0000", "bad-0000"))
                                       and "00001" not in n)]
    opened.append("model-00002-of-00003.gguf")
    golden = {"keys": keys, "files": {}}
    for name in sorted(opened):
        golden["files"][name] = reference_read(os.path.join(OUT, name), keys)
        print(name, golden["files"][name]["result"])
    with open(os.path.join(HERE, "gguf_ref.json"), "w") as f:
        json.dump(golden, f, indent=1, sort_keys=True)


if __name__ == "__main__":
    main()

"""GGUF v3 tensor table (include/edgexpu_gguf_upload.h) on synthetic files
written from the format's definition (tests/gguf_writer.py): the directory the
reference's loader builds (src/gguf.c:359-610) -- names, dims, types,
offsets relative to the data section, the data section at the end of the
infos rounded up to 32 whatever general.alignment declares (src/gguf.c:595
never reads that key) -- and the loader's refusals, including element counts
and byte sizes that overflow 64 bits.  No GPU."""
import numpy as np
import pytest

import edgexpu_amd as E
import gguf_writer as G
from edgexpu_amd import synth


@pytest.fixture(scope="module")
def gg():
    return E.Gguf()


def _model(rng):
    return [("token_embd.weight", [576, 40], E.Q8_0, synth.np_weights(E.Q8_0, 40, 576, rng)),
            ("blk.0.attn_q.weight", [4096, 16], E.Q4_K, synth.np_weights(E.Q4_K, 16, 4096, rng)),
            ("blk.0.ffn_down.weight", [2560, 7], E.Q6_K, synth.np_weights(E.Q6_K, 7, 2560, rng)),
            ("output_norm.weight", [576], E.F32, rng.normal(0, 1, 576).astype(np.float32)),
            ("blk.0.attn_k.weight", [256, 3], E.Q5_K, synth.np_weights(E.Q5_K, 3, 256, rng))]


KVS = [("general.architecture", G.STRING, "llama"), ("general.name", G.STRING, "synthetic"),
       ("llama.block_count", G.U32, 1), ("llama.rope.freq_base", G.F32, 10000.0),
       ("tokenizer.ggml.tokens", G.ARRAY, (G.STRING, ["<s>", "</s>", "a", "bb" * 40])),
       ("tokenizer.ggml.scores", G.ARRAY, (G.F32, [0.0, -1.5, 2.0])),
       ("some.nested", G.ARRAY, (G.ARRAY, [(G.U16, [1, 2, 3]), (G.STRING, ["x", "yz"])])),
       ("flag", G.BOOL, 1), ("i64", G.I64, -5), ("f64", G.F64, 2.5), ("u8", G.U8, 7), ("i16", G.I16, -3)]


@pytest.mark.parametrize("alignment", [None, 32, 64])
def test_table_matches_the_written_file(gg, tmp_path, alignment):
    rng = np.random.default_rng(1 + (alignment or 0))
    tensors = _model(rng)
    path = str(tmp_path / "m.gguf")
    kvs = KVS if alignment != 64 else KVS + [("pad", G.STRING, "p" * 39)]
    data_offset, offsets, info_end = G.write_gguf(path, kvs, [(n, d, t, G.as_bytes(a)) for n, d, t, a in tensors],
                                                  alignment=alignment)
    tab = gg.read_table(path)
    assert tab["version"] == 3
    assert tab["alignment"] == (alignment or 32)
    assert tab["kv_count"] == len(kvs) + (alignment is not None)
    assert tab["tensor_count"] == len(tensors)
    # the reference's data offset: the end of the infos rounded up to 32
    assert tab["data_offset"] == -(-info_end // 32) * 32
    if alignment == 64:
        # a file laid out for 64 whose infos end in the first half of a
        # 64-byte line: the data the writer put at the next 64 lies 32 bytes
        # past where the reference (and this reader) start the section
        assert info_end % 64 < 32 and data_offset == tab["data_offset"] + 32
        return
    assert tab["data_offset"] == data_offset
    for (name, dims, t, arr), off, got in zip(tensors, offsets, tab["tensors"]):
        assert got["name"] == name and got["dims"] == dims and got["type"] == t and got["offset"] == off
        assert got["nbytes"] == arr.nbytes
    raw = open(path, "rb").read()
    for (_, _, _, arr), got in zip(tensors, tab["tensors"]):
        lo = tab["data_offset"] + got["offset"]
        assert raw[lo:lo + got["nbytes"]] == G.as_bytes(arr)


def test_long_names_are_truncated_like_the_reference(gg, tmp_path):
    """A tensor name of 120 bytes keeps its first 95 (read_string_into into a
    96-byte field); the table stays aligned."""
    rng = np.random.default_rng(3)
    long = "blk.0." + "x" * 114
    w = synth.np_weights(E.Q8_0, 2, 64, rng)
    path = str(tmp_path / "n.gguf")
    G.write_gguf(path, [], [(long, [64, 2], E.Q8_0, G.as_bytes(w)), ("b", [64, 2], E.Q8_0, G.as_bytes(w))])
    tab = gg.read_table(path)
    assert tab["tensors"][0]["name"] == long[:95]
    assert tab["tensors"][1]["name"] == "b"


@pytest.mark.parametrize("case", ["magic", "version", "truncated_kv", "truncated_infos", "dims", "past_end",
                                  "overflow_elements", "overflow_bytes", "missing"])
def test_refusals(gg, tmp_path, case):
    rng = np.random.default_rng(4)
    w = synth.np_weights(E.Q4_K, 4, 256, rng)
    path = str(tmp_path / f"{case}.gguf")
    if case == "missing":
        with pytest.raises(ValueError, match="cannot open"):
            gg.read_table(path)
        return
    if case == "dims":
        G.write_gguf(path, [], [("t", [256, 1, 1, 1, 4], E.Q4_K, G.as_bytes(w))])
        with pytest.raises(ValueError, match="more than 4 dims"):
            gg.read_table(path)
        return
    if case in ("overflow_elements", "overflow_bytes"):
        # Q4_K dims whose product wraps to 256 in 64 bits, and F32 dims whose
        # element count fits but whose byte size (x 4) does not
        dims = [2 ** 56 + 1, 256] if case == "overflow_elements" else [2 ** 31, 2 ** 31]
        G.write_gguf(path, [], [("t", dims, E.Q4_K if case == "overflow_elements" else E.F32, G.as_bytes(w))])
        with pytest.raises(ValueError, match="overflows 64 bits"):
            gg.read_table(path)
        return
    if case == "version":
        G.write_gguf(path, [], [("t", [256, 4], E.Q4_K, G.as_bytes(w))], version=2)
        with pytest.raises(ValueError, match="version 3"):
            gg.read_table(path)
        return
    data_offset, _, _ = G.write_gguf(path, KVS, [("t", [256, 4], E.Q4_K, G.as_bytes(w))])
    raw = bytearray(open(path, "rb").read())
    if case == "magic":
        raw[0:4] = b"GGML"
        msg = "not a GGUF"
    elif case == "truncated_kv":
        raw = raw[:40]
        msg = "metadata"
    elif case == "truncated_infos":
        raw = raw[:data_offset - 40]
        msg = "tensor"
    else:  # past_end: the data section is cut
        raw = raw[:data_offset + w.nbytes - 1]
        msg = "past the end"
    open(path, "wb").write(bytes(raw))
    with pytest.raises(ValueError, match=msg):
        gg.read_table(path)

"""CPU: the GGUF tensor index (fl_gguf_*, host code of libloki_moe) on files written by tests/_gguf.py: tensor offsets,
types, dims and bytes, the expert stride ggml_row_size(type, ne0) * ne1 (src/server_core_fused.cpp:305), metadata of
every value type, several files (a later file's tensor replaces an earlier one, as the reference's index map,
src/server_core_fused.cpp:97-110), and rejection of malformed files."""
import numpy as np
import pytest

from tests import _gguf
from tests.golden import gen


def loki():
    import loki_amd
    if not __import__("os").path.exists(loki_amd.LIB_PATH):
        pytest.skip("libloki_moe.so not built")
    return loki_amd


def sample_tensors(seed=5):
    rng = np.random.default_rng(seed)
    t = []
    t.append(("blk.3.ffn_norm.weight", "F32", [512], rng.normal(size=512).astype(np.float32).view(np.uint8)))
    t.append(("blk.3.exp_probs_b.bias", "F32", [4], rng.normal(size=4).astype(np.float32).view(np.uint8)))
    t.append(("blk.3.ffn_gate_inp_f16.weight", "F16", [512, 4], rng.normal(size=2048).astype(np.float16).view(np.uint8)))
    t.append(("blk.3.ffn_gate_exps.weight", "IQ2_XXS", [512, 64, 3], gen.iq2_matrix(1, 2, 64 * 3, 512)))
    t.append(("blk.3.ffn_down_exps.weight", "Q3_K", [256, 96, 3], gen.kq_matrix(1, 3, 6, 96 * 3, 256)))
    t.append(("blk.3.ffn_down_shexp.weight", "Q6_K", [256, 96], gen.kq_matrix(1, 4, 1, 96, 256)))
    t.append(("token_embd.weight", "Q8_0", [64, 10], rng.integers(0, 256, 10 * 2 * 34, dtype=np.uint8)))
    return t


KV = [("general.architecture", "str", "deepseek2"), ("deepseek2.expert_count", "u32", 256),
      ("deepseek2.expert_used_count", "i32", 8), ("deepseek2.expert_weights_scale", "f32", 2.5),
      ("deepseek2.leading_dense_block_count", "u64", 3), ("x.i8", "i8", -5), ("x.u16", "u16", 65000), ("x.i16", "i16", -300),
      ("x.i64", "i64", -(1 << 40)), ("x.f64", "f64", 0.1), ("x.bool", "bool", True), ("x.u8", "u8", 200),
      ("tokenizer.ggml.tokens", "arr", ("str", ["<s>", "</s>", "hello"])), ("x.scores", "arr", ("f32", [0.5, 1.5]))]


@pytest.mark.parametrize("alignment", [None, 64])
def test_index_matches_written_file(tmp_path, alignment):
    lk = loki()
    path = str(tmp_path / "a.gguf")
    ts = sample_tensors()
    offs = _gguf.write(path, ts, KV, alignment=alignment)
    g = lk.Gguf(path)
    assert g.names() == [t[0] for t in ts]
    for name, tn, ne, raw in ts:
        t = g.tensor(name)
        assert t.file == 0 and t.offset == offs[name] and t.type == _gguf.GGML[tn][0] and t.n_dims == len(ne)
        assert list(t.ne)[:len(ne)] == ne and all(v == 1 for v in list(t.ne)[len(ne):])
        assert t.nbytes == len(raw) and t.row_bytes == _gguf.row_bytes(tn, ne[0])
        assert np.array_equal(g.read(name), raw)
        if t.offset % (alignment or 32):
            pytest.fail("unaligned tensor offset")
    # a slice, and the expert stride of expert tensors (eng:305)
    t = g.tensor("blk.3.ffn_down_exps.weight")
    es = t.row_bytes * t.ne[1]
    raw = dict((n, r) for n, _, _, r in ts)["blk.3.ffn_down_exps.weight"]
    assert es == 96 * 110 and np.array_equal(g.read("blk.3.ffn_down_exps.weight", 2 * es, es), raw[2 * es:3 * es])
    assert t.fl_format == lk.FL_Q3K and g.tensor("blk.3.ffn_gate_exps.weight").fl_format == lk.FL_IQ2
    assert g.tensor("blk.3.ffn_down_shexp.weight").fl_format == lk.FL_Q6K and g.tensor("blk.3.ffn_norm.weight").fl_format == -1
    with pytest.raises(KeyError):
        g.tensor("blk.4.ffn_norm.weight")
    # metadata
    assert g.get_str("general.architecture") == "deepseek2"
    assert g.get_int("deepseek2.expert_count") == 256 and g.get_int("deepseek2.expert_used_count") == 8
    assert g.get_int("deepseek2.leading_dense_block_count") == 3 and g.get_int("x.i8") == -5 and g.get_int("x.u16") == 65000
    assert g.get_int("x.i16") == -300 and g.get_int("x.i64") == -(1 << 40) and g.get_int("x.bool") == 1 and g.get_int("x.u8") == 200
    assert g.get_float("deepseek2.expert_weights_scale") == 2.5 and g.get_float("x.f64") == 0.1
    assert g.get_int("general.architecture") is None and g.get_float("nope") is None and g.get_str("x.u8") is None
    g.close()


def test_several_files(tmp_path):
    """two shards: tensors of both are indexed with their file; a repeated name takes the later file's tensor"""
    lk = loki()
    ts = sample_tensors()
    a, b = str(tmp_path / "s1.gguf"), str(tmp_path / "s2.gguf")
    _gguf.write(a, ts[:4], KV[:2])
    newer = ("blk.3.ffn_norm.weight", "F32", [512], np.arange(512, dtype=np.float32).view(np.uint8))
    offs_b = _gguf.write(b, ts[4:] + [newer], [("general.architecture", "str", "other")])
    g = lk.Gguf([a, b])
    assert sorted(g.names()) == sorted(t[0] for t in ts)
    assert g.tensor("blk.3.ffn_gate_exps.weight").file == 0 and g.tensor("blk.3.ffn_down_exps.weight").file == 1
    t = g.tensor("blk.3.ffn_norm.weight")
    assert t.file == 1 and t.offset == offs_b["blk.3.ffn_norm.weight"]
    assert np.array_equal(g.read("blk.3.ffn_norm.weight").view(np.float32), np.arange(512, dtype=np.float32))
    assert g.get_str("general.architecture") == "deepseek2"   # metadata: the first file's value
    g.close()


def test_rejects_malformed(tmp_path):
    lk = loki()
    ts = sample_tensors()[:3]
    good = str(tmp_path / "good.gguf")
    _gguf.write(good, ts, KV[:3])
    data = open(good, "rb").read()
    cases = {
        "magic": b"GGUX" + data[4:],
        "version": data[:4] + (1).to_bytes(4, "little") + data[8:],
        "truncated infos": data[:200],
        "truncated data": data[:-16],
    }
    for why, blob in cases.items():
        p = str(tmp_path / ("bad_%s.gguf" % why.replace(" ", "_")))
        open(p, "wb").write(blob)
        with pytest.raises(lk.LokiError):
            lk.Gguf(p)
    with pytest.raises(lk.LokiError):
        lk.Gguf(str(tmp_path / "missing.gguf"))
    # an offset that is not a multiple of the alignment
    p = str(tmp_path / "misaligned.gguf")
    _gguf.write(p, ts, KV[:3], alignment=64)
    blob = bytearray(open(p, "rb").read())
    name = ts[1][0].encode()
    i = blob.index(name) + len(name) + 4 + 8 * len(ts[1][2]) + 4   # that tensor's offset field
    blob[i:i + 8] = (8).to_bytes(8, "little")
    open(p, "wb").write(bytes(blob))
    with pytest.raises(lk.LokiError):
        lk.Gguf(p)
    lk.Gguf(good).close()


def test_rejects_wrapping_sizes_and_offsets(tmp_path):
    """A tensor whose byte size overflows 64 bits (dims each within the 2^40 limit) and one whose offset wraps when the
    data section's base is added are rejected, not indexed with a wrapped size that passes the end-of-file test."""
    lk = loki()
    ts = [("blk.0.ffn_gate_exps.weight", "IQ2_XXS", [512, 64, 3], gen.iq2_matrix(1, 2, 64 * 3, 512))]
    good = str(tmp_path / "g.gguf")
    _gguf.write(good, ts)
    data = bytearray(open(good, "rb").read())
    name = ts[0][0].encode()
    dims = data.index(name) + len(name) + 4                      # ne[0..2], then type, then offset
    huge = bytearray(data)
    for d in (1, 2):                                             # 64 * 3 rows -> 2^40 x 2^40: the product wraps
        huge[dims + 8 * d:dims + 8 * d + 8] = (1 << 40).to_bytes(8, "little")
    p = str(tmp_path / "huge.gguf")
    open(p, "wb").write(bytes(huge))
    with pytest.raises(lk.LokiError):
        lk.Gguf(p)
    wrap = bytearray(data)
    off = dims + 8 * 3 + 4
    wrap[off:off + 8] = ((1 << 64) - 32 * 8).to_bytes(8, "little")   # aligned; + the data base wraps past 2^64
    p = str(tmp_path / "wrap.gguf")
    open(p, "wb").write(bytes(wrap))
    with pytest.raises(lk.LokiError):
        lk.Gguf(p)

"""The GGUF container and the model mapping (host side of qr_gguf_*) against
the reference's own gguf_init_from_buffer (src/gguf.c:50-177) and
load_transformer / load_gguf_transformer (src/model.c:253-481), both compiled
from the reference's sources into oracle/_ref: the same files accepted and
refused, the same tensor table and data offsets, the same key/value lookups,
the same configuration and the same weight pointers.  Host only (no GPU)."""
import os
import struct

import numpy as np
import pytest

import gguf_writer as G
import inputs as I
import quantr_amd as Q

REF = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle", "_ref",
                   "libqref_c99.so")
pytestmark = pytest.mark.skipif(not os.path.exists(REF), reason="needs oracle/_ref (make -C oracle ref)")


@pytest.fixture(scope="module")
def ref():
    from oracle import RefLib
    return RefLib("c99")


def _ours(data):
    try:
        g = Q.Gguf(data)
    except Q.QrError:
        return None
    h = g.info()
    ts = []
    for t in g.tensors():
        t = dict(t)
        t["offset"] = t.pop("data") - g.base
        ts.append(t)
    g.close()
    return h, ts


def _files():
    a = I.decode_model("a")
    b = I.decode_model("b")
    c = I.decode_model("c")
    dd = I.decode_model("d")
    q3 = I.qwen3_small_model(n_layers=1, seq_len=64)
    at = dict(a)
    at["wcls"], at["wcls_type"] = a["tok_embd"], a["tok_type"]
    return {
        "a_tied": G.decode_model_gguf(
            at, mutate=lambda ts: [t for t in ts if t[0] != "output.weight"])[0],
        "a": G.decode_model_gguf(a)[0],
        "b_no_tokens": G.decode_model_gguf(b, tokens=False)[0],
        "q3_split_align64": G.decode_model_gguf(q3, split_experts=True, alignment=64,
                                                head_dim_key=True)[0],
        "c_dense": G.decode_model_gguf(c)[0],
        "d_dense_align64": G.decode_model_gguf(dd, alignment=64)[0],
    }


FILES = _files()


@pytest.mark.parametrize("name", sorted(FILES))
def test_parse_matches_reference(ref, name):
    data = FILES[name]
    want = ref.gguf_parse(data)
    got = _ours(data)
    assert want is not None and got is not None
    assert got[0] == want[0]
    assert len(got[1]) == len(want[1])
    for g, w in zip(got[1], want[1]):
        assert g == w, (g, w)


def test_truncations_refused_like_reference(ref):
    """Every prefix of a file's header (and a little past it): both parsers
    accept or refuse it alike, and agree on what they accept."""
    data = FILES["q3_split_align64"]
    hdr = ref.gguf_parse(data)[0]["data_offset"]
    for cut in list(range(0, hdr + 96, 3)) + [len(data) - 1, len(data)]:
        want = ref.gguf_parse(data[:cut])
        got = _ours(data[:cut])
        assert (want is None) == (got is None), cut
        if want is not None:
            assert got[0] == want[0] and got[1] == want[1], cut


def _raw(kv_bytes, n_kv, tensor_bytes=b"", n_t=0, magic=b"GGUF", version=3, tail=b"\0" * 64):
    return magic + struct.pack("<IQQ", version, n_t, n_kv) + kv_bytes + tensor_bytes + tail


def _s(x):
    return struct.pack("<Q", len(x)) + x


MALFORMED = {
    "bad_magic": _raw(b"", 0, magic=b"GGUX"),
    "version_7": _raw(b"", 0, version=7),
    "kv_count_65537": _raw(b"", 65537),
    "kv_count_65536_short": _raw(b"", 65536),
    "tensor_count_65537": _raw(b"", 0, n_t=65537),
    "kv_unknown_type": _raw(_s(b"k") + struct.pack("<I", 13) + b"\0" * 8, 1),
    "kv_string_too_long": _raw(_s(b"k") + struct.pack("<IQ", 8, 1024 * 1024 + 1) + b"x" * 64, 1),
    "kv_string_1mib": _raw(_s(b"k") + struct.pack("<IQ", 8, 1024 * 1024) + b"x" * (1024 * 1024), 1),
    "arr_1000001": _raw(_s(b"k") + struct.pack("<IIQ", 9, 0, 1000001) + b"\0" * 64, 1),
    "arr_unknown_elem": _raw(_s(b"k") + struct.pack("<IIQ", 9, 9, 1) + b"\0" * 64, 1),
    "arr_past_end": _raw(_s(b"k") + struct.pack("<IIQ", 9, 4, 100), 1, tail=b"\0" * 12),
    "alignment_zero": _raw(_s(b"general.alignment") + struct.pack("<II", 4, 0), 1),
    "alignment_u64": _raw(_s(b"general.alignment") + struct.pack("<IQ", 10, 128), 1),
    "alignment_wrong_type": _raw(_s(b"general.alignment") + struct.pack("<If", 6, 64.0), 1),
    "n_dims_5": _raw(b"", 0, _s(b"t") + struct.pack("<I", 5) + b"\0" * 48, 1),
    "n_dims_4": _raw(b"", 0, _s(b"t") + struct.pack("<I4QIQ", 4, 1, 1, 1, 1, 0, 0), 1),
    "tensor_past_end": _raw(b"", 0, _s(b"t") + struct.pack("<IQIQ", 1, 4, 0, 1 << 20), 1),
    "tensor_at_end": _raw(b"", 0, _s(b"t") + struct.pack("<IQIQ", 1, 4, 0, 32), 1),
}


@pytest.mark.parametrize("name", sorted(MALFORMED))
def test_malformed_like_reference(ref, name):
    data = MALFORMED[name]
    want = ref.gguf_parse(data)
    got = _ours(data)
    assert (want is None) == (got is None), (name, want, got)
    if want is not None:
        assert got == want


def test_values_match_reference(ref):
    data = FILES["a"]
    g = Q.Gguf(data)
    keys = ["general.architecture", "qwen3moe.embedding_length", "qwen3moe.block_count",
            "qwen3moe.rope.freq_base", "qwen3moe.expert_count", "tokenizer.ggml.tokens",
            "missing.key"]
    for k in keys:
        u, f, s = ref.gguf_vals(data, k, 7, -1.5)
        assert g.u32(k, 7) == u, k
        assert np.float32(g.f32(k, -1.5)) == np.float32(f), k
        assert (g.str(k) or "") == s, k
    assert g.arr_len("tokenizer.ggml.tokens") == 300
    assert g.arr_len("missing.key") == -1
    g.close()


@pytest.mark.parametrize("name", ["a", "a_tied", "b_no_tokens", "q3_split_align64", "c_dense",
                                  "d_dense_align64"])
def test_model_mapping_matches_reference(ref, tmp_path, name):
    """load_transformer's configuration and every weight pointer (as a file
    offset) against qr_gguf_model_host / qr_gguf_expert_host."""
    data = FILES[name]
    path = str(tmp_path / "m.gguf")
    open(path, "wb").write(data)
    g = Q.Gguf(data)
    mm, layers = g.model_host(seq_len=64)
    L, E = mm.n_layers, layers[0].moe.n_experts
    cfg, rope, off, types, rb = ref.load_gguf(path, L, E)
    dim, hidden, nl, H, KVH, vocab, seq, ne, K = [int(v) for v in cfg]
    assert (dim, nl, H, KVH, ne, K) == (mm.dim, L, mm.n_heads, mm.n_kv_heads, E,
                                        layers[0].moe.n_used)
    assert hidden == layers[0].moe.hidden
    assert np.float32(rope) == np.float32(mm.rope_base)
    if g.arr_len("tokenizer.ggml.tokens") > 0:
        assert vocab == mm.vocab  # otherwise the reference assumes 152064; ours reads the rows
    if g.u32("qwen3moe.attention.key_length", 0) == 0:
        assert mm.head_dim == dim // H
    b = g.base
    o = lambda p: -1 if p is None else p - b  # noqa: E731
    want = [o(mm.tok_embd), o(mm.rms_final), o(mm.wcls)]
    want_t = [mm.tok_type, mm.wcls_type]
    for y in layers:
        want += [o(y.rms_att), o(y.rms_ffn), o(y.wq), o(y.wk), o(y.wv), o(y.wo), o(y.moe.router)]
        want_t += [y.wq_type, y.wk_type, y.wv_type, y.wo_type, y.moe.up_type, y.moe.down_type,
                   y.moe.gate_type]
    for l in range(L):
        if E == 0:  # a dense layer: w1, w2, w3 in the expert fields
            y = layers[l].moe
            want += [y.up - b, y.down - b, y.gate - b]
        for e in range(E):
            up, down, gate = g.expert_host(l, e)
            want += [up - b, down - b, gate - b]
    assert list(off) == want
    assert list(types) == want_t
    if name == "a_tied":
        assert mm.wcls == mm.tok_embd
    assert rb == Q.load().qr_row_bytes(mm.tok_type, mm.dim)
    g.close()


def _edit(name, fn):
    def mutate(ts):
        return [fn(t) if t[0] == name else t for t in ts]
    return mutate


@pytest.mark.parametrize("case,match", [
    ("router_width", "ffn_gate_inp"),
    ("norm_quantized", "attn_norm"),
    ("q_rows", "attn_q"),
    ("expert_missing", "expert"),
    ("unknown_type", "attn_k"),
])
def test_model_host_refuses_bad_shapes(case, match):
    """Shapes and types are checked before anything is uploaded (the reference
    trusts them): a router of the wrong width, a norm stored quantized, a q
    projection of the wrong height, a missing expert tensor, a type the
    decoder has no kernel for."""
    m = I.decode_model("a")
    Q.Gguf(G.decode_model_gguf(m)[0]).model_host()
    if case == "router_width":
        mut = _edit("blk.1.ffn_gate_inp.weight", lambda t: (t[0], t[1], [128, t[2][1]], t[3]))
    elif case == "norm_quantized":
        mut = _edit("blk.0.attn_norm.weight", lambda t: (t[0], 8, t[2], t[3]))
    elif case == "q_rows":
        mut = _edit("blk.0.attn_q.weight", lambda t: (t[0], t[1], [t[2][0], t[2][1] // 2], t[3]))
    elif case == "expert_missing":
        def mut(ts):
            return [t for t in ts if t[0] != "blk.1.ffn_down_exps.weight"]
    else:
        mut = _edit("blk.1.attn_k.weight", lambda t: (t[0], 2, t[2], t[3]))
    data = G.decode_model_gguf(m, mutate=mut)[0]
    with pytest.raises(Q.QrError, match=match):
        Q.Gguf(data).model_host()


@pytest.mark.parametrize("key,value", [("embedding_length", 1 << 21), ("expert_count", 5000),
                                       ("expert_feed_forward_length", 1 << 21)])
def test_model_host_refuses_sizes_beyond_limits(key, value):
    """Widths and counts whose products (rows x row bytes x experts) could
    approach size_t's range are refused before any size arithmetic."""
    m = I.decode_model("a")
    data, _ = G.decode_model_gguf(m)
    kv = ("qwen3moe.%s" % key).encode()
    i = data.index(kv) + len(kv) + 4  # the key's u32 value after its type
    data = data[:i] + struct.pack("<I", value) + data[i + 4:]
    with pytest.raises(Q.QrError, match="limits|shape|expert"):
        Q.Gguf(data).model_host()


@pytest.mark.parametrize("case", ["type", "rows", "past_end"])
def test_expert_host_checks_each_expert(case):
    """Per-expert tensors beyond expert 0 (which the mapping checks) are
    checked when they are looked up for the gather: expert 1 of another type,
    of other dimensions, or whose bytes run past the end of the file is
    refused; expert 0 and the other experts still resolve."""
    m = I.decode_model("a")
    name = "blk.1.ffn_down_exps.1.weight"
    if case == "type":
        mut = _edit(name, lambda t: (t[0], 8, t[2], t[3]))
    elif case == "rows":
        mut = _edit(name, lambda t: (t[0], t[1], [t[2][0], t[2][1] * 2], t[3]))
    else:
        def mut(ts):
            # expert 1's down tensor last, with no bytes: its data starts at the end
            mine = [t for t in ts if t[0] == name][0]
            return [t for t in ts if t[0] != name] + [(mine[0], mine[1], mine[2], b"")]
    data, _ = G.decode_model_gguf(m, split_experts=True, mutate=mut)
    g = Q.Gguf(data)
    g.model_host()
    g.expert_host(1, 0)
    g.expert_host(1, 2)
    with pytest.raises(Q.QrError, match="expert_host"):
        g.expert_host(1, 1)
    g.close()

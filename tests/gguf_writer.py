"""A minimal GGUF (version 3) writer for tests: the container format that
gguf_init_from_buffer (src/gguf.c:50-177) parses, written from the published
format (little-endian; header, key/value pairs, tensor infos, padding to the
alignment, tensor data at aligned offsets).  Test infrastructure only."""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?",
        U64: "<Q", I64: "<q", F64: "<d"}


def _str(s):
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _value(t, v):
    if t == STR:
        return _str(v)
    if t == ARR:
        et, items = v
        out = struct.pack("<IQ", et, len(items))
        for it in items:
            out += _value(et, it)
        return out
    return struct.pack(_FMT[t], v)


def gguf_bytes(kvs, tensors, alignment=32, version=3, put_alignment_kv=False):
    """kvs: list of (key, type, value); array values are (elem_type, items).
    tensors: list of (name, ggml_type, ne (innermost first), data bytes).
    Returns the file's bytes."""
    kv = list(kvs)
    if put_alignment_kv:
        kv.append(("general.alignment", U32, alignment))
    out = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kv))
    for k, t, v in kv:
        out += _str(k) + struct.pack("<I", t) + _value(t, v)
    offs, off = [], 0
    for name, typ, ne, data in tensors:
        offs.append(off)
        off += len(data)
        off = (off + alignment - 1) // alignment * alignment
    for (name, typ, ne, data), o in zip(tensors, offs):
        out += _str(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", n) for n in ne)
        out += struct.pack("<IQ", typ, o)
    pad = (-len(out)) % alignment
    out += b"\0" * pad
    base = len(out)
    blob = bytearray(off)
    for (name, typ, ne, data), o in zip(tensors, offs):
        blob[o:o + len(data)] = data
    return bytes(out) + bytes(blob), base


def decode_model_gguf(m, arch="qwen3moe", alignment=32, split_experts=False, tokens=True,
                      head_dim_key=False, mutate=None):
    """A decode model dict (tests/golden/inputs.py decode_model /
    qwen3_small_model) as GGUF tensors with the names load_gguf_transformer
    reads (src/model.c:253-449).  expert_w1 (the SiLU slot) is
    ffn_up_exps, expert_w3 ffn_gate_exps, expert_w2 ffn_down_exps; a dense
    model (E = 0) has ffn_up (w1), ffn_gate (w3) and ffn_down (w2).  mutate
    (optional) edits the (name, type, ne, bytes) list before it is written."""
    dim, L, E, hid, V = m["dim"], m["n_layers"], m["E"], m["hidden"], m["vocab"]
    H, KVH, hd = m["n_heads"], m["n_kv_heads"], m["head_dim"]
    kvs = [("general.architecture", STR, arch),
           ("%s.embedding_length" % arch, U32, dim),
           ("%s.block_count" % arch, U32, L),
           ("%s.attention.head_count" % arch, U32, H),
           ("%s.attention.head_count_kv" % arch, U32, KVH)]
    if E > 0:
        kvs += [("%s.expert_count" % arch, U32, E),
                ("%s.expert_used_count" % arch, U32, m["K"]),
                ("%s.expert_feed_forward_length" % arch, U32, hid)]
    else:  # a dense model: no expert keys, feed_forward_length (src/model.c:283-296)
        kvs.append(("%s.feed_forward_length" % arch, U32, hid))
    kvs.append(("%s.rope.freq_base" % arch, F32, float(m["rope_base"])))
    if head_dim_key:
        kvs.append(("%s.attention.key_length" % arch, U32, hd))
    if tokens:
        kvs.append(("tokenizer.ggml.tokens", ARR, (STR, ["t%d" % i for i in range(V)])))
    b = lambda a: np.ascontiguousarray(a).tobytes()  # noqa: E731
    t = [("token_embd.weight", m["tok_type"], [dim, V], b(m["tok_embd"])),
         ("output_norm.weight", 0, [dim], b(m["rms_final"])),
         ("output.weight", m["wcls_type"], [dim, V], b(m["wcls"]))]
    wt = m["wtype"]
    for l, lw in enumerate(m["layers"]):
        p = "blk.%d." % l
        t += [(p + "attn_norm.weight", 0, [dim], b(lw["rms_att"])),
              (p + "ffn_norm.weight", 0, [dim], b(lw["rms_ffn"])),
              (p + "attn_q.weight", wt[0], [dim, H * hd], b(lw["wq"])),
              (p + "attn_k.weight", wt[1], [dim, KVH * hd], b(lw["wk"])),
              (p + "attn_v.weight", wt[2], [dim, KVH * hd], b(lw["wv"])),
              (p + "attn_output.weight", wt[3], [H * hd, dim], b(lw["wo"]))]
        ut, dt = m["up_type"], m["down_type"]
        up, gate, down = b(lw["up"]), b(lw["gate"]), b(lw["down"])
        if E == 0:  # the dense FFN's tensors (src/model.c:434-446)
            t += [(p + "ffn_up.weight", ut, [dim, hid], up),
                  (p + "ffn_down.weight", dt, [hid, dim], down),
                  (p + "ffn_gate.weight", ut, [dim, hid], gate)]
            continue
        t.append((p + "ffn_gate_inp.weight", 0, [dim, E], b(lw["router"])))
        if split_experts:
            su, sd = len(up) // E, len(down) // E
            for e in range(E):
                t += [(p + "ffn_up_exps.%d.weight" % e, ut, [dim, hid], up[e * su:(e + 1) * su]),
                      (p + "ffn_down_exps.%d.weight" % e, dt, [hid, dim], down[e * sd:(e + 1) * sd]),
                      (p + "ffn_gate_exps.%d.weight" % e, ut, [dim, hid], gate[e * su:(e + 1) * su])]
        else:
            t += [(p + "ffn_up_exps.weight", ut, [dim, hid, E], up),
                  (p + "ffn_down_exps.weight", dt, [hid, dim, E], down),
                  (p + "ffn_gate_exps.weight", ut, [dim, hid, E], gate)]
    if mutate is not None:
        t = mutate(t)
    return gguf_bytes(kvs, t, alignment=alignment, put_alignment_kv=alignment != 32)

"""The .cmf v2 reader (csrc/container.cpp through the C ABI, cmf_amd.container)
and the Qwen3 loader (cmf_amd.loader), on the CPU.  Mirrors the reference's
container tests (crates/cortiq-core/tests/roundtrip.rs): hash64 cross-vectors,
full-file round trip, page alignment of large tensors, strict rejection of
garbage and corruption, verify() locating a flipped byte; plus sharded
opens, directory edge cases and the loader's mapping of a model file."""
import struct

import numpy as np
import pytest

import cmf_writer as W


def _mod():
    from cmf_amd import container
    return container


# ---------------------------------------------------------------- hash64
VECTORS = [(b"", 0x0), (b"CMF", 0xB59AA39A074033EC), (b"0123456789abcdef", 0x30D401310062EA9F),
           (bytes(range(256)), 0x9955BB876C0706BF)]  # roundtrip.rs:227-233


@pytest.mark.parametrize("data,want", VECTORS)
def test_hash64_reference_vectors(data, want):
    assert W.hash64_py(data) == want  # the test-side restatement
    assert _mod().hash64(data) == want  # the library's


def test_hash64_native_matches_restatement_on_ragged_lengths():
    rng = np.random.default_rng(3)
    for n in list(range(0, 40)) + [1000, 4097]:
        b = rng.integers(0, 256, n, dtype=np.uint8).tobytes()
        assert _mod().hash64(b) == W.hash64_py(b), n


# ---------------------------------------------------------------- files
def _tiny_tensors():
    """roundtrip.rs:160-225: f32 embedding, q8_row and q4_block gate, f16 norm."""
    vocab, hidden, inter = 10, 8, 16
    embed = np.sin(np.arange(vocab * hidden, dtype=np.float32) * np.float32(0.13)).astype(np.float32)
    gate = np.cos(np.arange(inter * hidden, dtype=np.float32) * np.float32(0.07)).astype(np.float32)
    norm = (1.0 + np.arange(hidden, dtype=np.float32) * np.float32(0.01)).astype(np.float32)
    q4 = bytes(range(18)) * (inter * hidden // 32)
    return [("model.embed_tokens.weight", 0, (vocab, hidden), embed.tobytes()),
            ("model.layers.0.mlp.gate_proj.weight", 3, (inter, hidden), W.encode_q8_row(gate, inter, hidden)),
            ("model.layers.1.mlp.gate_proj.weight", 4, (inter, hidden), q4),
            ("model.norm.weight", 1, (hidden,), W.f16_bytes(norm))]


def _tiny_header():
    a = {"arch_name": "tiny-test", "hidden_size": 8, "intermediate_size": 16, "num_layers": 2,
         "num_attention_heads": 2, "num_kv_heads": 1, "head_dim": 4, "vocab_size": 10,
         "layer_types": ["FullAttention"] * 2, "rms_norm_eps": 1e-6, "norm_style": "qwen",
         "rope_theta": 10000.0, "tie_word_embeddings": False, "max_position_embeddings": 64}
    return W.header_of(a)


VOCAB = b'{"model":{"type":"BPE","vocab":{},"merges":[]}}'
MASKS = bytes(range(7)) * 5  # opaque section bytes: only their hash is checked here


def _write_tiny(path, **kw):
    kw.setdefault("masks", MASKS)
    kw.setdefault("vocab", VOCAB)
    return W.write(path, _tiny_header(), _tiny_tensors(), **kw)


def test_full_file_roundtrip(tmp_path):
    p = tmp_path / "tiny.cmf"
    _write_tiny(p)
    f = _mod().CmfFile.open(p)
    assert f.header["version"] == 2
    assert f.arch["arch_name"] == "tiny-test"
    specs = _tiny_tensors()
    assert len(f.tensors) == len(specs)
    for (name, dt, shape, data), e in zip(specs, f.tensors):
        assert e.name == name and e.dtype == dt and e.shape == shape
        assert e.off % 64 == 0
        assert bytes(f.tensor_bytes(name)) == data
        assert f.tensor(name) is e or f.tensor(name).index == e.index
    assert f.verify() == []
    assert f.vocab == VOCAB
    assert bytes(f.section_bytes("masks")) == MASKS
    assert f.required_features == W.F_TENSOR_DIR | W.F_BINARY_MASKS
    assert f.tensor("no.such.tensor") is None
    with pytest.raises(_mod().MissingTensor):
        f.tensor_bytes("no.such.tensor")
    f.close()


def test_large_tensors_are_page_aligned(tmp_path):
    """roundtrip.rs:352-397"""
    rows, cols = 512, 64
    vals = np.sin(np.arange(rows * cols, dtype=np.float32) * np.float32(0.01)).astype(np.float32)
    big = W.encode_q8_row(vals, rows, cols)
    t = [("big.weight", 3, (rows, cols), big), ("small.norm", 1, (8,), W.f16_bytes(1 + np.arange(8)))]
    p = tmp_path / "align.cmf"
    W.write(p, _tiny_header(), t)
    f = _mod().CmfFile.open(p)
    e = f.tensor("big.weight")
    assert e.nbytes >= 16 * 1024 and e.off % 4096 == 0
    assert all(x.off % 64 == 0 for x in f.tensors)
    assert bytes(f.tensor_bytes("big.weight")) == big
    assert f.verify() == []


def _patch(path, pos, b):
    raw = bytearray(open(path, "rb").read())
    raw[pos:pos + len(b)] = b
    open(path, "wb").write(bytes(raw))


def test_open_rejects_garbage_and_corruption(tmp_path):
    """roundtrip.rs:399-492"""
    K = _mod()
    g = tmp_path / "garbage.bin"
    g.write_bytes(b"not a cmf, definitely not a 27B model")
    with pytest.raises((K.InvalidMagic, K.BoundsError)):
        K.CmfFile.open(g)
    s = tmp_path / "small.bin"
    s.write_bytes(b"CMF\x01")
    with pytest.raises(K.BoundsError):
        K.CmfFile.open(s)
    with pytest.raises(K.FileNotFound):
        K.CmfFile.open(tmp_path / "absent.cmf")

    # header tamper inside a JSON string: opens, verify names the header
    p = tmp_path / "tamper.cmf"
    _write_tiny(p)
    raw = open(p, "rb").read()
    i = raw.index(b'"cmf"')
    _patch(p, i + 2, b"x")
    f = K.CmfFile.open(p)
    assert any("section 'header'" in x for x in f.verify())
    f.close()

    p = tmp_path / "v.cmf"
    _write_tiny(p)
    _patch(p, 4, b"\x01")
    with pytest.raises(K.UnsupportedVersion, match="1"):
        K.CmfFile.open(p)

    p = tmp_path / "f.cmf"
    _write_tiny(p)
    raw = open(p, "rb").read()
    _patch(p, 12, bytes([raw[12] | 0x80]))
    with pytest.raises(K.UnsupportedFeature, match="128"):
        K.CmfFile.open(p)

    p = tmp_path / "dir-overflow.cmf"
    _write_tiny(p)
    dir_off = struct.unpack_from("<Q", open(p, "rb").read(), 0x20)[0]
    _patch(p, dir_off, struct.pack("<Q", (1 << 64) - 1))
    with pytest.raises(K.ParseError):
        K.CmfFile.open(p)

    p = tmp_path / "t.cmf"
    _write_tiny(p)
    raw = open(p, "rb").read()
    p.write_bytes(raw[: len(raw) // 2])
    with pytest.raises(K.BoundsError):
        K.CmfFile.open(p)

    # a flipped weight byte: exactly one problem, naming the tensor
    p = tmp_path / "h.cmf"
    _write_tiny(p)
    f = K.CmfFile.open(p)
    assert f.verify() == []
    off = f.tensor("model.embed_tokens.weight").off
    f.close()
    data_off = struct.unpack_from("<Q", open(p, "rb").read(), 0x30)[0]
    raw = open(p, "rb").read()
    _patch(p, data_off + off, bytes([raw[data_off + off] ^ 0xFF]))
    f = K.CmfFile.open(p)
    probs = f.verify()
    assert len(probs) == 1 and "embed_tokens" in probs[0]


def test_section_hash_mismatch_and_malformed(tmp_path):
    K = _mod()
    p = tmp_path / "s.cmf"
    _write_tiny(p)
    voff = struct.unpack_from("<Q", open(p, "rb").read(), 0x50)[0]
    raw = open(p, "rb").read()
    _patch(p, voff, bytes([raw[voff] ^ 1]))
    f = K.CmfFile.open(p)
    probs = f.verify()
    assert len(probs) == 1 and probs[0].startswith("section 'vocab': hash mismatch")
    f.close()
    # a malformed stored hex string is reported, not raised
    p2 = tmp_path / "m.cmf"
    h = _tiny_header()
    h["section_hashes"] = {"vocab": "zz"}
    t = _tiny_tensors()
    W.write(p2, h, t)
    # writer added no section_hashes (no optional sections): the header's own
    # entry stays as written
    f = K.CmfFile.open(p2)
    assert f.verify() == ["section 'vocab': malformed hash 'zz'"]


def _dir_file(tmp_path, mutate):
    """A tiny file whose directory record 0 is rewritten by mutate(bytearray,
    rec_off); the envelope's dir hash is left stale (open() does not check it)."""
    p = tmp_path / "d.cmf"
    _write_tiny(p)
    raw = bytearray(open(p, "rb").read())
    dir_off = struct.unpack_from("<Q", raw, 0x20)[0]
    mutate(raw, dir_off + 16)
    p.write_bytes(bytes(raw))
    return p


def test_directory_validation(tmp_path):
    K = _mod()
    cases = [
        (lambda r, o: r.__setitem__(slice(o + 6, o + 7), bytes([99])), K.UnknownDtype),   # dtype id
        (lambda r, o: r.__setitem__(slice(o + 7, o + 8), bytes([7])), K.ParseError),      # ndim 7
        (lambda r, o: struct.pack_into("<Q", r, o + 32, 8), K.BoundsError),               # off % 64
        (lambda r, o: struct.pack_into("<Q", r, o + 40, 1 << 40), K.BoundsError),         # past data
        (lambda r, o: struct.pack_into("<I", r, o + 8, 11), K.BoundsError),               # nbytes != expected
        (lambda r, o: struct.pack_into("<I", r, o, 1 << 20), K.ParseError),               # name out of pool
    ]
    for mut, exc in cases:
        with pytest.raises(exc):
            K.CmfFile.open(_dir_file(tmp_path, mut))


def test_duplicate_and_non_utf8_names(tmp_path):
    K = _mod()
    t = _tiny_tensors()
    p = tmp_path / "dup.cmf"
    W.write(p, _tiny_header(), t + [t[3]])
    with pytest.raises(K.ParseError, match="duplicate"):
        K.CmfFile.open(p)
    p = tmp_path / "utf.cmf"
    W.write(p, _tiny_header(), [("abé", 1, (8,), W.f16_bytes(np.ones(8)))])
    raw = bytearray(open(p, "rb").read())
    i = raw.index("abé".encode())
    raw[i + 2] = 0xC3  # 0xC3 0xC3: broken sequence
    raw[i + 3] = 0xC3
    p.write_bytes(bytes(raw))
    with pytest.raises(K.ParseError, match="UTF-8"):
        K.CmfFile.open(p)


def test_header_must_be_a_json_object_with_required_fields(tmp_path):
    K = _mod()
    p = tmp_path / "j.cmf"
    _write_tiny(p)
    raw = open(p, "rb").read()
    i = raw.index(b'"format"')
    _patch(p, i, b"{")  # breaks the JSON syntax
    with pytest.raises(K.ParseError):
        K.CmfFile.open(p)
    h = _tiny_header()
    del h["quant_type"]
    p = tmp_path / "k.cmf"
    W.write(p, h, _tiny_tensors())
    with pytest.raises(K.ParseError, match="quant_type"):
        K.CmfFile.open(p)


def test_data_section_must_be_page_aligned(tmp_path):
    K = _mod()
    p = tmp_path / "a.cmf"
    _write_tiny(p)
    raw = open(p, "rb").read()
    data_off = struct.unpack_from("<Q", raw, 0x30)[0]
    _patch(p, 0x30, struct.pack("<Q", data_off - 64))
    with pytest.raises(K.BoundsError, match="aligned"):
        K.CmfFile.open(p)


def test_open_sharded_merges_directories(tmp_path):
    """format.rs:589-650: shard 1 carries the coordinates, siblings by name."""
    K = _mod()
    t = _tiny_tensors()
    h1, h2 = _tiny_header(), _tiny_header()
    h1["shard"] = {"no": 1, "count": 2}
    h2["shard"] = {"no": 2, "count": 2}
    W.write(tmp_path / "m-00001-of-00002.cmf", h1, t[:2])
    W.write(tmp_path / "m-00002-of-00002.cmf", h2, t[2:])
    f = K.CmfFile.open_sharded(tmp_path / "m-00001-of-00002.cmf")
    assert [e.name for e in f.tensors] == [x[0] for x in t]
    assert [e.shard for e in f.tensors] == [0, 0, 1, 1]
    for name, dt, shape, data in t:
        assert bytes(f.tensor_bytes(name)) == data
    assert f.verify() == []
    # plain file: open_sharded == open
    _write_tiny(tmp_path / "plain.cmf")
    assert len(K.CmfFile.open_sharded(tmp_path / "plain.cmf").tensors) == 4
    # wrong entry shard, duplicate across shards, wrong coordinates
    with pytest.raises(K.ParseError, match="open shard 1"):
        K.CmfFile.open_sharded(tmp_path / "m-00002-of-00002.cmf")
    W.write(tmp_path / "d-00001-of-00002.cmf", h1, t[:2])
    W.write(tmp_path / "d-00002-of-00002.cmf", h2, t[1:])
    with pytest.raises(K.ParseError, match="across shards"):
        K.CmfFile.open_sharded(tmp_path / "d-00001-of-00002.cmf")
    h3 = _tiny_header()
    h3["shard"] = {"no": 3, "count": 2}
    W.write(tmp_path / "w-00001-of-00002.cmf", h1, t[:2])
    W.write(tmp_path / "w-00002-of-00002.cmf", h3, t[2:])
    with pytest.raises(K.ParseError, match="wrong shard coords"):
        K.CmfFile.open_sharded(tmp_path / "w-00001-of-00002.cmf")
    with pytest.raises(K.FileNotFound):
        W.write(tmp_path / "x-00001-of-00003.cmf", dict(h1, shard={"no": 1, "count": 3}), t[:2])
        K.CmfFile.open_sharded(tmp_path / "x-00001-of-00003.cmf")


# ---------------------------------------------------------------- loader
TINY = dict(n_layers=2, hidden=256, n_heads=4, n_kv=2, head_dim=128, inter=512, vocab=512, max_seq=128,
            rope_theta=1e6, eps=1e-6)


def _same_tensor(a, b):
    assert a["dtype"] == b["dtype"] and a["rows"] == b["rows"] and a["cols"] == b["cols"]
    if a["dtype"] == 3:
        assert np.array_equal(np.asarray(a["q"]), np.asarray(b["q"]))
        assert np.array_equal(np.asarray(a["row_scale"], np.float32), np.asarray(b["row_scale"], np.float32))
    else:
        assert bytes(np.asarray(a["bytes"], np.uint8)) == bytes(np.asarray(b["bytes"], np.uint8))


def _same_layer(a, b):
    for k in a:
        if k == "moe":
            ma, mb = a["moe"], b["moe"]
            assert (ma["top_k"], ma["norm_topk"]) == (mb["top_k"], mb["norm_topk"])
            _same_tensor(ma["router"], mb["router"])
            assert len(ma["experts"]) == len(mb["experts"])
            for ea, eb in zip(ma["experts"], mb["experts"]):
                for n in ("gate", "up", "down"):
                    _same_tensor(ea[n], eb[n])
        elif isinstance(a[k], dict):
            _same_tensor(a[k], b[k])
        else:
            assert np.array_equal(np.asarray(a[k], np.float32), np.asarray(b[k], np.float32)), k


@pytest.mark.parametrize("norm_dtype", [0, 1, 2])
def test_loader_maps_a_model_file(tmp_path, norm_dtype):
    from cmf_amd import synth, loader
    sm = W.f16_model(synth.synth_model(TINY, seed=3, norm_noise=0.1))
    if norm_dtype:  # the norms as the file holds them
        cast = {1: lambda v: np.asarray(v, np.float32).astype(np.float16).astype(np.float32),
                2: lambda v: np.frombuffer(W.bf16_bytes(v), "<u2").astype(np.uint32).__lshift__(16).view(np.float32)}
        c = cast[norm_dtype]
        for l in sm["layers"] + [sm["mtp"]["layer"]]:
            for k in ("input_norm", "post_norm", "q_norm", "k_norm"):
                l[k] = c(l[k])
        sm["final_norm"] = c(sm["final_norm"])
        for k in ("enorm", "hnorm", "norm"):
            sm["mtp"][k] = c(sm["mtp"][k])
    p = tmp_path / "model.cmf"
    W.write_model(p, sm, norm_dtype)
    m = loader.load(str(p))
    assert m["cfg"] == dict(TINY)
    for a, b in zip(sm["layers"], m["layers"]):
        _same_layer(a, b)
    _same_tensor(sm["lm_head"], m["lm_head"])
    assert "embed" not in m  # tied
    assert np.array_equal(sm["final_norm"], m["final_norm"])
    for k in ("enorm", "hnorm", "norm"):
        assert np.array_equal(sm["mtp"][k], m["mtp"][k])
    _same_tensor(sm["mtp"]["eh_proj"], m["mtp"]["eh_proj"])
    _same_layer(sm["mtp"]["layer"], m["mtp"]["layer"])
    assert m["file"].verify() == []


def test_loader_untied_embedding_and_q4tp(tmp_path):
    from cmf_amd import synth, loader
    sm = W.f16_model(synth.synth_model(TINY, seed=4, mtp=False))
    sm["embed"] = W.round_q8_scales(synth.q8_normal(77, TINY["vocab"], TINY["hidden"]))
    sm["layers"][1]["down"] = synth.q4tp_uniform(78, TINY["hidden"], TINY["inter"])
    p = tmp_path / "u.cmf"
    W.write_model(p, sm)
    m = loader.load(str(p), max_seq=64)
    assert m["cfg"]["max_seq"] == 64
    _same_tensor(sm["embed"], m["embed"])
    _same_tensor(sm["lm_head"], m["lm_head"])
    _same_tensor(sm["layers"][1]["down"], m["layers"][1]["down"])
    assert "mtp" not in m


@pytest.mark.parametrize("router", ["f16", "q8"])
def test_loader_moe_layers(tmp_path, router):
    from cmf_amd import CmfError
    """Qwen3-MoE blocks (build_ffn_at's MoE arm, loader.rs:~200-400): the
    router `mlp.gate.weight` (f16 as the reference converter stores it, or
    q8) and `mlp.experts.{e}.*` by presence; arch.moe gives top_k and
    norm_topk_prob; the loaded model runs the oracle forward as the memory one"""
    from cmf_amd import synth, loader
    from oracle import oracle as orc
    moe = dict(n_experts=6, top_k=2, inter=64, layers=[1], router_dtype=router)
    sm = W.f16_model(synth.synth_model(TINY, seed=6, norm_noise=0.1, moe=moe))
    p = tmp_path / "moe.cmf"
    W.write_model(p, sm)
    m = loader.load(str(p))
    for a, b in zip(sm["layers"], m["layers"]):
        _same_layer(a, b)
    assert "moe" in m["layers"][1] and "moe" not in m["layers"][0]
    toks = synth.ids(7, 3, TINY["vocab"])
    a = [orc.OracleModel(sm, threads=2).forward(int(toks[0]), 0)]
    b = [orc.OracleModel(m, threads=2).forward(int(toks[0]), 0)]
    assert np.array_equal(a[0], b[0])
    # what the engine does not run is refused by name
    W.write_model(p, sm, moe={"num_experts": 6, "top_k": 2, "moe_intermediate_size": 64, "router_sigmoid": True})
    with pytest.raises(CmfError, match="router_sigmoid"):
        loader.load(str(p))


def test_loader_refuses_what_the_engine_cannot_run(tmp_path):
    from cmf_amd import CmfError, synth, loader
    sm = W.f16_model(synth.synth_model(TINY, seed=5, mtp=False))
    p = tmp_path / "r.cmf"
    W.write_model(p, sm, sliding_window=128)
    with pytest.raises(CmfError, match="sliding_window"):
        loader.load(str(p))
    W.write_model(p, sm, layer_types=["FullAttention", "LinearAttention"])
    with pytest.raises(CmfError, match="full-attention"):
        loader.load(str(p))
    # a matrix format without an MI355X kernel
    t = W.model_tensors(sm)
    t = [(n, 4, s, bytes(len(b) and ((s[0] * s[1] + 31) // 32) * 18)) if n.endswith("layers.0.mlp.up_proj.weight")
         else (n, d, s, b) for n, d, s, b in t]
    W.write(p, W.header_of(W.arch_of(TINY, mtp=False)), t)
    with pytest.raises(CmfError, match="q4_block"):
        loader.load(str(p))
    # untied without lm_head
    t = [x for x in W.model_tensors(sm)]
    W.write(p, W.header_of(W.arch_of(TINY, mtp=False, tie=False)), t)
    with pytest.raises(CmfError, match="lm_head"):
        loader.load(str(p))


def test_corrupted_files_fail_cleanly(tmp_path):
    """Random byte damage (biased to the envelope and directory) either opens
    or raises a CmfFileError; an opened file's views and verify() stay usable."""
    K = _mod()
    p = tmp_path / "seed.cmf"
    _write_tiny(p)
    seed = open(p, "rb").read()
    rng = np.random.default_rng(11)
    q = tmp_path / "fz.cmf"
    opened = 0
    for it in range(400):
        b = bytearray(seed)
        for _ in range(int(rng.integers(1, 8))):
            lim = [128, 2176, len(b)][int(rng.integers(0, 3))]
            pos = int(rng.integers(0, min(lim, len(b))))
            b[pos] = int(rng.integers(0, 256))
        if rng.integers(0, 10) == 0:
            b = b[: int(rng.integers(0, len(b) + 1))]
        q.write_bytes(bytes(b))
        try:
            f = K.CmfFile.open(q)
        except K.CmfFileError:
            continue
        opened += 1
        for e in f.tensors:
            assert len(f.entry_bytes(e)) == e.nbytes
        assert isinstance(f.verify(), list)
        f.close()
    assert opened > 0

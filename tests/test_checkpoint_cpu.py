"""The checkpoint reader and the loader's conversions (libtgohip.so through its C
ABI) against the reference's own known answers: every refusal row of
safetensors/safetensors_test.go and repo_test.go (the message fragments are the
reference's), and the decode / transpose / head-permutation vectors of
weights/convert_test.go. CPU only."""
import json
import os

import numpy as np
import pytest

import tgo_amd
from stwrite import bf16_bits, build, good, write, write_arrays, write_index, write_raw


def refuse_open(path, want):
    with pytest.raises(tgo_amd.TgoError) as e:
        tgo_amd.SafeTensors(path)
    assert want in str(e.value), (str(e.value), want)


def mutated(tmp_path, mutate, length=None):
    hdr, data = good()
    mutate(hdr)
    return write(str(tmp_path / "model.safetensors"), hdr, data, length)


# safetensors_test.go:269-415 (TestRefusals), one row each.
REFUSALS = [
    ("end before begin", lambda h: h["a"].update(data_offsets=[16, 0]),
     "a: data_offsets end 0 is before begin 16"),
    ("offsets past the data region", lambda h: h["b"].update(data_offsets=[16, 1024]),
     "b: data_offsets [16,1024) lie outside"),
    ("negative begin", lambda h: h["a"].update(data_offsets=[-16, 0]),
     "a: data_offsets [-16,0) lie outside"),
    ("data_offsets has one element", lambda h: h["a"].update(data_offsets=[0]),
     "a: data_offsets has 1 elements"),
    ("overlapping tensors", lambda h: h["b"].update(data_offsets=[12, 18], shape=[3]),
     "b [12,18) overlaps a [0,16)"),
    ("shape disagrees with the byte span", lambda h: h["a"].update(shape=[2, 3]),
     "a: shape [2 3] of dtype F32 needs 24 bytes, but data_offsets span 16"),
    ("unknown dtype", lambda h: h["a"].update(dtype="F8_E4M3"), 'a: unknown dtype "F8_E4M3"'),
    ("negative dimension", lambda h: h["a"].update(shape=[2, -2]),
     "a: shape dimension 1 is negative (-2)"),
    ("shape product overflows", lambda h: h["a"].update(shape=[1 << 40, 1 << 40]),
     "a: shape [1099511627776 1099511627776] is larger than this platform can index"),
    ("element count times width overflows", lambda h: h["a"].update(dtype="F64", shape=[1 << 62]),
     "a: shape [4611686018427387904] of dtype F64 is larger than this platform can index"),
    ("entry is not an object", lambda h: h.update(a=7), "a: parse entry"),
    ("metadata is not a map of strings", lambda h: h.update(__metadata__={"total_size": 22}),
     "__metadata__ is not a map of strings"),
]


@pytest.mark.parametrize("name,mutate,want", REFUSALS, ids=[r[0] for r in REFUSALS])
def test_reader_refuses_what_the_reference_refuses(tmp_path, name, mutate, want):
    refuse_open(mutated(tmp_path, mutate), want)


def test_header_length_refusals(tmp_path):
    refuse_open(mutated(tmp_path, lambda h: None, length=1 << 20), "exceeds the")
    tgo_amd.set_safetensors_header_cap(4)
    try:
        refuse_open(mutated(tmp_path, lambda h: None), "byte limit")
    finally:
        tgo_amd.set_safetensors_header_cap(0)
    tgo_amd.SafeTensors(mutated(tmp_path, lambda h: None)).close()


def test_short_and_unparseable_files(tmp_path):
    for body in (b"", b"1234567"):  # safetensors_test.go:417-448
        p = tmp_path / "short"
        p.write_bytes(body)
        refuse_open(str(p), "shorter than the 8-byte header length")
    _, data = good()
    for js in (b"[1,2,3]", b"{oops"):
        refuse_open(write_raw(str(tmp_path / "j"), js, data), "parse header")


def test_open_reads_header_and_planes(tmp_path):
    path = write(str(tmp_path / "m.safetensors"), *good())
    with tgo_amd.SafeTensors(path) as f:
        ent = f.entries()
        assert list(ent) == ["a", "b"]  # name order; __metadata__ is not a tensor
        assert ent["a"] == ("F32", (2, 2), 0, 16) and ent["b"] == ("BF16", (3,), 16, 22)
        assert f.read("a") == b"\x11" * 16 and f.read("b") == b"\x22" * 6
        with pytest.raises(tgo_amd.TgoError, match="nope"):
            f.read("nope")


def test_padding_empty_and_scalar_tensors(tmp_path):
    hdr, data = good()
    js = json.dumps(hdr, separators=(",", ":")).encode()
    while (8 + len(js)) % 8:
        js += b" "
    js += b" " * 8  # safetensors_test.go:463-495: a whole extra block of padding
    with tgo_amd.SafeTensors(write_raw(str(tmp_path / "p"), js, data)) as f:
        assert f.entries()["a"][2] == 0 and f.read("a") == b"\x11" * 16
    # An empty tensor owns no bytes and cannot overlap (safetensors_test.go:170-190).
    hdr, data = build(("a", "F32", [2], 0x11), ("e", "F32", [0, 4], 0))
    hdr["e"]["data_offsets"] = [0, 0]
    with tgo_amd.SafeTensors(write(str(tmp_path / "e"), hdr, data)) as f:
        assert f.entries()["e"] == ("F32", (0, 4), 0, 0)
    # A scalar has shape [] and one element (safetensors_test.go:192-203).
    hdr, data = build(("s", "F32", [], 0x11))
    with tgo_amd.SafeTensors(write(str(tmp_path / "s"), hdr, data)) as f:
        assert f.entries()["s"] == ("F32", (), 0, 4)


def sharded(tmp_path):
    """repo_test.go:15-33: "a" in the first shard, "b" in the second."""
    d = str(tmp_path)
    (tmp_path / "config.json").write_text('{"architectures":["Qwen3ForCausalLM"]}')
    write(os.path.join(d, "model-00001-of-00002.safetensors"), *build(("a", "F32", [2, 2], 0x11)))
    write(os.path.join(d, "model-00002-of-00002.safetensors"), *build(("b", "BF16", [3], 0x22)))
    wm = {"a": "model-00001-of-00002.safetensors", "b": "model-00002-of-00002.safetensors"}
    write_index(d, wm)
    return d, wm


def refuse_repo(d, want):
    with pytest.raises(tgo_amd.TgoError) as e:
        tgo_amd.Repo(d)
    assert want in str(e.value), (str(e.value), want)


def test_repo_single_and_sharded(tmp_path):
    d, _ = sharded(tmp_path)
    with tgo_amd.Repo(d) as r:
        assert r.has("a") and r.has("b") and not r.has("c")
    single = tmp_path / "single"
    single.mkdir()
    write(str(single / "model.safetensors"), *good())
    with tgo_amd.Repo(str(single)) as r:  # no config.json is not a refusal
        assert r.has("a") and r.has("b")


def test_repo_refusals(tmp_path):  # repo_test.go:154-292
    empty = tmp_path / "empty"
    empty.mkdir()
    (empty / "config.json").write_text("{}")
    refuse_repo(str(empty), "no model.safetensors")
    bad = tmp_path / "badcfg"
    bad.mkdir()
    (bad / "config.json").write_text("{not json")
    write(str(bad / "model.safetensors"), *good())
    refuse_repo(str(bad), "not valid JSON")
    unr = tmp_path / "unreadable"
    unr.mkdir()
    (unr / "config.json").mkdir()
    refuse_repo(str(unr), "read config")
    unri = tmp_path / "unreadable_index"
    unri.mkdir()
    (unri / "model.safetensors.index.json").mkdir()
    refuse_repo(str(unri), "read index")

    def case(name, edit, want):
        sub = tmp_path / name
        sub.mkdir()
        d, wm = sharded(sub)
        edit(d, wm)
        refuse_repo(d, want)

    case("idxjson", lambda d, wm: open(os.path.join(d, "model.safetensors.index.json"), "w").write("{oops"),
         "parse index")
    case("nowm", lambda d, wm: write_index(d, None), "weight_map is empty or absent")
    case("missing", lambda d, wm: write_index(d, dict(wm, c="model-00003-of-00002.safetensors")),
         "c: shard model-00003-of-00002.safetensors is missing")
    case("absent", lambda d, wm: write_index(d, dict(wm, c=wm["a"])),
         "c: shard model-00001-of-00002.safetensors has no such tensor")
    case("moved", lambda d, wm: write_index(d, dict(wm, a=wm["b"])),
         "a: shard model-00002-of-00002.safetensors has no such tensor")
    case("malformed", lambda d, wm: open(os.path.join(d, wm["a"]), "wb").write(b"short"),
         "shorter than the 8-byte header length")
    stow = tmp_path / "stowaway"
    stow.mkdir()
    write(str(stow / "model-00001-of-00001.safetensors"),
          *build(("a", "F32", [2], 1), ("stowaway", "F32", [2], 2)))
    write_index(str(stow), {"a": "model-00001-of-00001.safetensors"})
    refuse_repo(str(stow), "stowaway in shard model-00001-of-00001.safetensors has no entry in the index")
    for i, shard in enumerate(["../secrets.safetensors", "sub/model.safetensors",
                               "..\\secrets.safetensors", "..", ".", ""]):
        case("esc%d" % i, lambda d, wm, s=shard: write_index(d, dict(wm, a=s)),
             "a: shard")
        sub = tmp_path / ("esc%d" % i)
        with pytest.raises(tgo_amd.TgoError, match="is not a file name in the model directory"):
            tgo_amd.Repo(str(sub))


def one_tensor_repo(tmp_path, name, dtype, arr):
    d = tmp_path / ("r_" + name)
    d.mkdir()
    write_arrays(str(d / "model.safetensors"), {name: (dtype, arr)})
    return tgo_amd.Repo(str(d))


def test_decode_bf16_is_a_shift(tmp_path):
    # convert_test.go:17-65: the nine patterns, then all 65536.
    cases = [(0x0000, 0x00000000), (0x8000, 0x80000000), (0x3f80, 0x3f800000),
             (0xbf80, 0xbf800000), (0x4049, 0x40490000), (0x7f80, 0x7f800000),
             (0xff80, 0xff800000), (0x0001, 0x00010000), (0x7f7f, 0x7f7f0000)]
    bits = np.array([c[0] for c in cases], np.uint16)
    with one_tensor_repo(tmp_path, "w", "BF16", bits) as r:
        got = r.plane("w", len(cases)).view(np.uint32)
    assert [int(x) for x in got] == [c[1] for c in cases]
    every = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    with one_tensor_repo(tmp_path, "all", "BF16", every) as r:
        got = r.plane("all", 65536).view(np.uint32)
    assert np.array_equal(got, np.arange(65536, dtype=np.uint32) << 16)


def test_decode_f16_f32_and_refusals(tmp_path):
    f16 = np.array([1, -2.5, 0.5, 2.0 ** -24, -65504, np.inf], np.float16)  # incl. a subnormal
    with one_tensor_repo(tmp_path, "h", "F16", f16.view(np.uint16)) as r:
        got = r.plane("h", 6)
    assert np.array_equal(got, f16.astype(np.float32))
    f32 = np.array([3, -4, 1e30], np.float32)
    with one_tensor_repo(tmp_path, "f", "F32", f32) as r:
        assert np.array_equal(r.plane("f", 3), f32)
    with one_tensor_repo(tmp_path, "i", "I64", np.zeros(1, np.int64)) as r:
        with pytest.raises(tgo_amd.TgoError, match="not a float plane"):
            r.plane("i", 1)


def test_transpose_and_head_permutation(tmp_path):
    # convert_test.go:261-281: [2,3] -> [3,2].
    m = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    with one_tensor_repo(tmp_path, "t", "F32", m) as r:
        assert list(r.plane("t", 6, transpose=True)) == [1, 4, 2, 5, 3, 6]
    # convert_test.go:283-295: two heads of four channels.
    x = np.array([[0, 1, 2, 3, 10, 11, 12, 13]], np.float32)
    with one_tensor_repo(tmp_path, "p", "F32", x) as r:
        assert list(r.plane("p", 8, head_dim=4)) == [0, 2, 1, 3, 10, 12, 11, 13]
        with pytest.raises(tgo_amd.TgoError, match="must be positive and even"):
            r.plane("p", 8, head_dim=3)
    with one_tensor_repo(tmp_path, "q", "F32", np.zeros((1, 6), np.float32)) as r:
        with pytest.raises(tgo_amd.TgoError, match="does not divide into heads"):
            r.plane("q", 6, head_dim=4)
    # convert_test.go:409-434: per head of each row, after the transpose.
    dh, heads, rows = 8, 3, 2
    w = np.arange(heads * dh * rows, dtype=np.float32).reshape(heads * dh, rows)  # [out, in]
    with one_tensor_repo(tmp_path, "w", "F32", w) as r:
        got = r.plane("w", w.size, transpose=True, head_dim=dh).reshape(rows, heads * dh)
    x = w.T  # [in, out]
    for seg in range(rows * heads):
        rr, h = divmod(seg, heads)
        for i in range(dh // 2):
            assert got[rr, h * dh + 2 * i] == x[rr, h * dh + i]
            assert got[rr, h * dh + 2 * i + 1] == x[rr, h * dh + i + dh // 2]


def test_bf16_checkpoint_round_trip(tmp_path):
    """A bf16 [out, in] projection comes back as exactly (bits << 16) transposed."""
    rng = np.random.default_rng(3)
    w = rng.standard_normal((16, 8)).astype(np.float32)
    b = bf16_bits(w)
    with one_tensor_repo(tmp_path, "x", "BF16", b) as r:
        got = r.plane("x", w.size, transpose=True).reshape(8, 16)
    want = (b.astype(np.uint32) << 16).view(np.float32).T
    assert np.array_equal(got, want)

"""XorSparse container (XORSPARE1) and the convert_sparse step.

CPU: the container bytes are pinned by hand against the documented layout
(SPARSE_FORMAT.md:30-50 / SparseFile::serialize, sparse_loader.rs:124-139):
magic, version at byte 9, count at byte 13, per-tensor header and blob; the
library writer equals the oracle's restatement of serialize byte for byte,
and the reader returns what was written (and rejects truncations, bad magic
and versions).  The reference reader's offset (version read at byte 8) is a
documented divergence: a file it would accept is shown to be one no
serialize call writes.  The converter's blob equals encode_sparse_tensor of
the destriped rows (and, with destripe off, of the reference converter's
linear unpack).  GPU: a layer built from a container entry computes exactly
what the dense Pack4 layer of the same checkpoint tensor computes.
"""
import struct

import numpy as np
import pytest

import oracle
import xtern


def rand_entries(rng, k=3):
    out = []
    for t in range(k):
        K, N = int(rng.integers(1, 300)), int(rng.integers(1, 40))
        tern = rng.integers(-1, 2, size=(N, K)).astype(np.int8)
        blob = oracle.sparse_encode_tensor(tern, K, N)[0]
        out.append((f"model.layers.{t}.mlp.down_proj.weight", N, K, float(np.float32(rng.random())),
                    blob))
    return out


def test_layout_by_hand():
    data = xtern.SparseFile.serialize([("w", 2, 3, 0.5, b"\x01\x02")])
    want = (b"XORSPARE1" + struct.pack("<I", 1) + struct.pack("<I", 1) + struct.pack("<I", 1) + b"w" +
            struct.pack("<I", 2) + struct.pack("<I", 3) + struct.pack("<f", 0.5) +
            struct.pack("<I", 2) + b"\x01\x02")
    assert data == want
    assert data[9:13] == b"\x01\x00\x00\x00" and data[13:17] == b"\x01\x00\x00\x00"
    # The reference reader takes the version from bytes 8..12: "1" + 3 bytes
    # of the real version field -> 0x31 + (1 << 8) = 0x131, not 1.
    assert struct.unpack_from("<I", data, 8)[0] == 0x131


def test_writer_matches_oracle_and_reader_roundtrips():
    rng = np.random.default_rng(1)
    ents = rand_entries(rng, 5)
    data = xtern.SparseFile.serialize(ents)
    assert data == oracle.sparse_container_serialize(ents)
    sf = xtern.SparseFile.from_bytes(data)
    assert len(sf) == 5
    parsed = oracle.sparse_container_parse(data)
    for i, (name, od, idim, ws, blob) in enumerate(ents):
        assert sf.entry(i) == (name, od, idim, np.float32(ws), blob)
        assert parsed[name] == (od, idim, np.float32(ws), blob)
        got_blob, got_ws = sf.get_sparse(name, idim, od)
        assert got_blob == blob and got_ws == np.float32(ws)
    with pytest.raises(xtern.XternError, match="not found"):
        sf.get_sparse("nope", 1, 1)
    name, od, idim, _, _ = ents[0]
    with pytest.raises(xtern.XternError, match="shape mismatch"):
        sf.get_sparse(name, idim + 1, od)


def test_duplicate_names_last_wins_and_empty_file():
    data = xtern.SparseFile.serialize([("a", 1, 1, 1.0, b"x"), ("a", 2, 2, 2.0, b"yy")])
    sf = xtern.SparseFile.from_bytes(data)
    assert sf.get_sparse("a", 2, 2) == (b"yy", 2.0)
    empty = xtern.SparseFile.serialize([])
    assert len(empty) == 17 and len(xtern.SparseFile.from_bytes(empty)) == 0


@pytest.mark.parametrize("cut", [0, 5, 16, 18, 22, 30, 40])
def test_reader_rejects_truncation(cut):
    data = xtern.SparseFile.serialize([("name", 4, 64, 1.0, bytes(20))])
    with pytest.raises(xtern.XternError):
        xtern.SparseFile.from_bytes(data[:cut])
    xtern.SparseFile.from_bytes(data)  # the whole file parses


def test_reader_rejects_bad_magic_and_version():
    data = bytearray(xtern.SparseFile.serialize([("n", 1, 1, 1.0, b"")]))
    bad = bytes(b"XORSPARE2" + data[9:])
    with pytest.raises(xtern.XternError, match="bad magic"):
        xtern.SparseFile.from_bytes(bad)
    data[9] = 2
    with pytest.raises(xtern.XternError, match="unsupported version 2"):
        xtern.SparseFile.from_bytes(bytes(data))


def stripe4(t):
    N, K = t.shape
    R = N // 4
    c = (t.astype(np.int64) + 1).reshape(4, R, K)
    return sum(c[j] << (2 * j) for j in range(4)).astype(np.uint8)


@pytest.mark.parametrize("K,N", [(64, 4), (100, 8), (2560, 640), (333, 20)])
def test_converter_blob(K, N):
    rng = np.random.default_rng(K + N)
    t = rng.integers(-1, 2, size=(N, K)).astype(np.int8)
    stored = stripe4(t)
    blob = xtern.hf_to_sparse_blob(xtern.XT_PACK4, K, N, stored)
    # destriped: the rows of the original matrix
    assert blob == oracle.sparse_encode_tensor(t, K, N)[0]
    assert blob == oracle.convert_sparse_tensor(stored, K, N, destripe=True)
    # reference converter: linear unpack of the stored bytes
    lin = xtern.hf_to_sparse_blob(xtern.XT_PACK4, K, N, stored, destripe=False)
    assert lin == oracle.convert_sparse_tensor(stored, K, N, destripe=False)
    if N > 4:
        assert lin != blob  # rows permuted, the divergence the destripe fixes


def test_converter_pack5_and_errors():
    rng = np.random.default_rng(3)
    K, N = 77, 15
    t = rng.integers(-1, 2, size=(N, K)).astype(np.int8)
    R = N // 5
    c = (t.astype(np.int64) + 1).reshape(5, R, K)
    stored = sum(c[j] * 3 ** j for j in range(5)).astype(np.uint8)
    assert xtern.hf_to_sparse_blob(xtern.XT_PACK5, K, N, stored) == \
        oracle.sparse_encode_tensor(t, K, N)[0]
    with pytest.raises(xtern.XternError, match="pre-packed U8"):
        xtern.hf_to_sparse_blob(xtern.XT_PACK4, K, 6, stored)


def test_convert_sparse_directory():
    rng = np.random.default_rng(4)
    t1 = rng.integers(-1, 2, size=(8, 64)).astype(np.int8)
    t2 = rng.integers(-1, 2, size=(4, 128)).astype(np.int8)
    tensors = {
        "model.layers.0.mlp.up_proj.weight": stripe4(t1),
        "model.layers.0.mlp.up_proj.weight_scale": np.array([2.0], np.float32),
        "model.layers.0.mlp.down_proj.weight": stripe4(t2),
        "model.layers.0.mlp.down_proj.weight_scale": np.array([0.25], np.float32),
        "model.embed_tokens.weight": np.zeros((4, 4), np.float32),  # not U8: skipped
        "model.norm.weight": np.zeros((2, 2), np.uint8),             # no scale: skipped
    }
    data = xtern.convert_sparse(tensors)
    sf = xtern.SparseFile.from_bytes(data)
    assert sorted(sf.names()) == ["model.layers.0.mlp.down_proj.weight",
                                  "model.layers.0.mlp.up_proj.weight"]
    blob, ws = sf.get_sparse("model.layers.0.mlp.up_proj.weight", 64, 8)
    assert blob == oracle.sparse_encode_tensor(t1, 64, 8)[0] and ws == np.float32(0.5)
    _, ws2 = sf.get_sparse("model.layers.0.mlp.down_proj.weight", 128, 4)
    assert ws2 == np.float32(4.0)
    data_noinv = xtern.convert_sparse(tensors, invert=False)
    assert xtern.SparseFile.from_bytes(data_noinv).get_sparse(
        "model.layers.0.mlp.up_proj.weight", 64, 8)[1] == np.float32(2.0)


@pytest.mark.gpu
@pytest.mark.parametrize("K,N", [(2560, 640), (4096, 1024), (333, 20)])
def test_layer_from_container_matches_dense(K, N):
    import torch
    print(f"[case] container layer K={K} N={N}", flush=True)
    rng = np.random.default_rng(K * N)
    t = rng.choice(np.array([-1, 0, 1], np.int8), size=(N, K), p=[0.3, 0.4, 0.3])
    stored = stripe4(t)
    name = "model.layers.3.self_attn.o_proj.weight"
    data = xtern.convert_sparse({name: stored, name + "_scale": np.array([1.7], np.float32)})
    sf = xtern.SparseFile.from_bytes(data)
    lin_s = xtern.TernaryLinear.from_sparse_file(sf, name, K, N)
    dw = sf.device_weights(name, K, N)
    lin_d = xtern.TernaryLinear.from_hf_prepacked(stored, K, N, xtern.TernaryPackType.Pack4, 1.7,
                                                  True)
    x = torch.from_numpy(rng.standard_normal((3, K)).astype(np.float32)).to("cuda:0")
    yd = lin_d.forward(x).cpu().numpy()
    assert np.array_equal(lin_s.forward(x).cpu().numpy().view(np.int32), yd.view(np.int32))
    assert np.array_equal(xtern.linear_f32(dw, x).cpu().numpy().view(np.int32), yd.view(np.int32))
    with pytest.raises(xtern.XternError, match="shape mismatch"):
        sf.device_weights(name, K, N + 1)

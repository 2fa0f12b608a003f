"""Expert containers: where each routed expert's six pieces lie in safetensors files
(mvllm_st_expert_pieces, host only), against fixtures written as the reference's tests
write them (tests/test_host.cpp:3636-3668, 3712-3735, 3817-3826) and by the safetensors
package.  The offsets are checked by reading the file there and comparing with the bytes
the fixture wrote."""
import json
import os
import struct

import numpy as np
import pytest

import mvllm_hip as hip
from st_fixture import make_container, piece_bytes, piece_name, write_st


def read_pieces(files, fi, off, nb):
    out = []
    for b in range(fi.shape[0]):
        parts = []
        for k in range(6):
            with open(files[fi[b, k]], "rb") as f:
                f.seek(int(off[b, k]))
                parts.append(f.read(int(nb[b, k])))
        out.append(b"".join(parts))
    return out


@pytest.mark.parametrize("fmt,D,I,prefix", [(4, 64, 64, "model."), (7, 32, 32, "")])
def test_reference_fixture_shapes(tmp_path, fmt, D, I, prefix):
    """The reference fixtures' shapes: GLM hidden 64 / intermediate 64, K3 32 x 32, two
    experts in layer 1 (first dense layer 0)."""
    rng = np.random.default_rng(fmt)
    blobs = make_container(str(tmp_path), rng, fmt, D, I, [1], 2, prefix)
    files, fi, off, nb = hip.st_expert_pieces(str(tmp_path), prefix, fmt, D, I, 1, 2, 2)
    assert len(files) == 1 and files[0].endswith("model.safetensors")
    assert (nb == np.array(piece_bytes(fmt, D, I))).all()
    got = read_pieces(files, fi, off, nb)
    assert got == [blobs[(1, 0)], blobs[(1, 1)]]
    geo = hip.expert_geom(fmt, D, I)
    assert len(got[0]) == geo[0]


def test_sharded_containers_and_layer_range(tmp_path):
    rng = np.random.default_rng(3)
    fmt, D, I = 7, 256, 128
    blobs = make_container(str(tmp_path), rng, fmt, D, I, [1, 2, 3], 4, "", n_files=3)
    files, fi, off, nb = hip.st_expert_pieces(str(tmp_path), "", fmt, D, I, 2, 4, 4)
    assert [os.path.basename(f) for f in files] == \
        [f"model-0000{i}-of-00003.safetensors" for i in (1, 2, 3)]
    assert len(set(fi.ravel().tolist())) > 1  # the pieces come from several files
    got = read_pieces(files, fi, off, nb)
    assert got == [blobs[(L, e)] for L in (2, 3) for e in range(4)]


def test_first_file_wins_and_other_files_ignored(tmp_path):
    """A name present in two containers resolves to the first in name order; files
    without the .safetensors suffix and directories are not read."""
    rng = np.random.default_rng(4)
    fmt, D, I = 4, 64, 64
    blobs = make_container(str(tmp_path / "a"), rng, fmt, D, I, [1], 1, "model.")
    other = make_container(str(tmp_path / "b"), rng, fmt, D, I, [1], 1, "model.")
    os.rename(tmp_path / "a" / "model.safetensors", tmp_path / "a" / "a.safetensors")
    os.rename(tmp_path / "b" / "model.safetensors", tmp_path / "a" / "b.safetensors")
    (tmp_path / "a" / "notes.txt").write_text("not a container")
    os.makedirs(tmp_path / "a" / "dir.safetensors")
    files, fi, off, nb = hip.st_expert_pieces(str(tmp_path / "a"), "model.", fmt, D, I, 1, 2, 1)
    assert [os.path.basename(f) for f in files] == ["a.safetensors", "b.safetensors"]
    assert read_pieces(files, fi, off, nb) == [blobs[(1, 0)]]
    assert blobs[(1, 0)] != other[(1, 0)]


def test_safetensors_package_container(tmp_path):
    """A container written by the safetensors package (header padded to 8 bytes,
    __metadata__ entry) with the pieces in another order than the blob order."""
    st = pytest.importorskip("safetensors.numpy")
    rng = np.random.default_rng(5)
    fmt, D, I = 7, 64, 64
    nbytes = piece_bytes(fmt, D, I)
    arrays, blob = {}, []
    for k in range(6):
        a = rng.integers(0, 256, nbytes[k], dtype=np.uint8)
        arrays[piece_name(fmt, "lm.", 0, 0, k)] = a
        blob.append(a.tobytes())
    st.save_file(arrays, str(tmp_path / "x.safetensors"), metadata={"format": "pt"})
    files, fi, off, nb = hip.st_expert_pieces(str(tmp_path), "lm.", fmt, D, I, 0, 1, 1)
    assert read_pieces(files, fi, off, nb) == [b"".join(blob)]


def test_json_escapes_in_names(tmp_path):
    """Names are JSON strings: escapes decode before the lookup."""
    fmt, D, I = 7, 32, 32
    nbytes = piece_bytes(fmt, D, I)
    tensors = [(piece_name(fmt, "", 1, 0, k), "U8", [nbytes[k]], bytes([k + 1]) * nbytes[k])
               for k in range(6)]
    header, o = {}, 0
    for name, dt, sh, data in tensors:
        header[name] = {"dtype": dt, "shape": sh, "data_offsets": [o, o + len(data)]}
        o += len(data)
    text = json.dumps(header, ensure_ascii=True).replace("model", "\\u006dodel").encode()
    with open(tmp_path / "m.safetensors", "wb") as f:
        f.write(struct.pack("<Q", len(text)) + text + b"".join(t[3] for t in tensors))
    files, fi, off, nb = hip.st_expert_pieces(str(tmp_path), "", fmt, D, I, 1, 2, 1)
    assert read_pieces(files, fi, off, nb) == [b"".join(t[3] for t in tensors)]


@pytest.mark.parametrize("fmt,msg", [(4, "glm53 expert pieces missing or wrong size at L1 E1"),
                                     (7, "k3 MXFP4 expert pieces missing or wrong size at L1 E1")])
def test_wrong_size_and_missing_piece(tmp_path, fmt, msg):
    rng = np.random.default_rng(6)
    D = I = 64
    prefix = "model." if fmt == 4 else ""
    make_container(str(tmp_path / "short"), rng, fmt, D, I, [1], 2, prefix)
    # the container holds I = 64 experts; asking for I = 128 makes every size wrong
    with pytest.raises(hip.HipError, match="wrong size at L1 E0"):
        hip.st_expert_pieces(str(tmp_path / "short"), prefix, fmt, D, 128, 1, 2, 2)
    # expert 1 missing its last piece
    from st_fixture import expert_tensors
    tensors, _ = expert_tensors(rng, fmt, D, I, [1], 2, prefix)
    os.makedirs(tmp_path / "miss")
    write_st(str(tmp_path / "miss" / "m.safetensors"), tensors[:-1])
    with pytest.raises(hip.HipError, match=msg):
        hip.st_expert_pieces(str(tmp_path / "miss"), prefix, fmt, D, I, 1, 2, 2)


def test_glm_float_codes_refused(tmp_path):
    rng = np.random.default_rng(7)
    make_container(str(tmp_path), rng, 4, 64, 64, [1], 1, "model.", code_dtype="F32")
    with pytest.raises(hip.HipError, match="glm53 f32 expert checkpoint"):
        hip.st_expert_pieces(str(tmp_path), "model.", 4, 64, 64, 1, 2, 1)


@pytest.mark.parametrize("case", ["zero_header", "huge_header", "not_object", "bad_json",
                                  "inverted", "no_dtype", "past_end", "no_dir",
                                  "huge_offset", "max_offset", "min_offset"])
def test_malformed_containers(tmp_path, case):
    fmt, D, I = 7, 32, 32
    nbytes = piece_bytes(fmt, D, I)
    tensors = [(piece_name(fmt, "", 0, 0, k), "U8", [nbytes[k]], bytes(nbytes[k]))
               for k in range(6)]
    path = tmp_path / "m.safetensors"
    write_st(str(path), tensors)
    raw = path.read_bytes()
    n = struct.unpack("<Q", raw[:8])[0]
    header = raw[8:8 + n].decode()
    expect = {"zero_header": "invalid safetensors header_size",
              "huge_header": "invalid safetensors header_size",
              "not_object": "not an object", "bad_json": "safetensors header",
              "inverted": "data_offsets inverted", "no_dtype": "missing dtype",
              "past_end": "past the end", "no_dir": "opendir",
              "huge_offset": "integer out of range", "max_offset": "wrong size",
              "min_offset": "data_offsets"}[case]
    if case == "zero_header":
        raw = struct.pack("<Q", 0) + raw[8:]
    elif case == "huge_header":
        raw = struct.pack("<Q", 200_000_000) + raw[8:]
    elif case == "not_object":
        h = ("[" + header[1:-1] + "]").encode()
        raw = struct.pack("<Q", len(h)) + h + raw[8 + n:]
    elif case == "bad_json":
        h = header[:-1].encode() + b",}"
        raw = struct.pack("<Q", len(h)) + h + raw[8 + n:]
    elif case == "inverted":
        d = json.loads(header)
        k = next(iter(d))
        d[k]["data_offsets"] = d[k]["data_offsets"][::-1]
        h = json.dumps(d).encode()
        raw = struct.pack("<Q", len(h)) + h + raw[8 + n:]
    elif case == "no_dtype":
        d = json.loads(header)
        del d[next(iter(d))]["dtype"]
        h = json.dumps(d).encode()
        raw = struct.pack("<Q", len(h)) + h + raw[8 + n:]
    elif case == "past_end":
        raw = raw[:-10]
    elif case in ("huge_offset", "max_offset", "min_offset"):
        # 19- and 20-digit offsets: out of the 64-bit range must be an error, not an
        # exception escaping the C entry point
        big = {"huge_offset": "9999999999999999999", "max_offset": "9223372036854775807",
               "min_offset": "-9223372036854775808"}[case]
        d = json.loads(header)
        k = next(iter(d))
        lo, hi = d[k]["data_offsets"]
        h = json.dumps(d).replace(f"[{lo}, {hi}]", f"[{lo}, {big}]" if case != "min_offset"
                                  else f"[{big}, {hi}]", 1).encode()
        raw = struct.pack("<Q", len(h)) + h + raw[8 + n:]
    path.write_bytes(raw)
    where = str(tmp_path / "absent") if case == "no_dir" else str(tmp_path)
    with pytest.raises(hip.HipError, match=expect):
        hip.st_expert_pieces(where, "", fmt, D, I, 0, 1, 1)

"""Safetensors expert containers for the loader tests, written the way the reference's
tests write theirs (write_safetensors_file, tests/test_host.cpp:3636-3668: header JSON
with tensors in order and data offsets back to back, no padding), or with the
safetensors package (8-byte header padding, __metadata__)."""
import json
import os
import struct

import numpy as np

GLM_PIECES = ["gate_proj.weight", "gate_proj.weight.qs", "up_proj.weight", "up_proj.weight.qs",
              "down_proj.weight", "down_proj.weight.qs"]


def write_st(path, tensors, metadata=None):
    """tensors: list of (name, dtype, shape, bytes).  Reference layout (no padding)."""
    header, off = {}, 0
    if metadata is not None:
        header["__metadata__"] = metadata
    for name, dtype, shape, data in tensors:
        header[name] = {"dtype": dtype, "shape": list(shape),
                        "data_offsets": [off, off + len(data)]}
        off += len(data)
    text = json.dumps(header, separators=(",", ":")).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(text)))
        f.write(text)
        for _, _, _, data in tensors:
            f.write(data)


def piece_bytes(fmt, D, I):
    """Byte counts of the six pieces in blob (and name) order."""
    if fmt == 4:
        pg, sg = I * ((D + 1) // 2), I * ((D + 63) // 64) * 4
        pd, sd = D * ((I + 1) // 2), D * ((I + 63) // 64) * 4
        return [pg, sg, pg, sg, pd, sd]
    pg, sg = I * ((D + 1) // 2), I * ((D + 31) // 32)
    pd, sd = D * ((I + 1) // 2), D * ((I + 31) // 32)
    return [pg, sg, pd, sd, pg, sg]  # w1 (gate), w2 (down), w3 (up)


def piece_name(fmt, prefix, L, e, k):
    if fmt == 4:
        return f"{prefix}layers.{L}.mlp.experts.{e}.{GLM_PIECES[k]}"
    mat, half = ("w1", "w2", "w3")[k // 2], ("packed", "scale")[k & 1]
    return f"{prefix}model.layers.{L}.block_sparse_moe.experts.{e}.{mat}.weight_{half}"


def piece_data(rng, fmt, nbytes, k):
    """Valid operands: random codes; int4 scales f32 in [0.005, 0.02]; MXFP4 scale bytes in
    [118, 124] (the bench's distributions)."""
    if k % 2 == 0:
        return rng.integers(0, 256, nbytes, dtype=np.uint8).tobytes()
    if fmt == 4:
        return rng.uniform(0.005, 0.02, nbytes // 4).astype(np.float32).tobytes()
    return rng.integers(118, 125, nbytes, dtype=np.uint8).tobytes()


def expert_tensors(rng, fmt, D, I, layers, n_experts, prefix, code_dtype="U8"):
    """-> (tensors, blobs): the container tensors of the given layers' experts, and each
    (layer, expert)'s expected blob (six pieces back to back)."""
    nb = piece_bytes(fmt, D, I)
    tensors, blobs = [], {}
    for L in layers:
        for e in range(n_experts):
            parts = []
            for k in range(6):
                data = piece_data(rng, fmt, nb[k], k)
                parts.append(data)
                if fmt == 4 and k % 2 == 1:
                    dtype, shape = "F32", [nb[k] // 4]
                else:
                    dtype, shape = (code_dtype if k % 2 == 0 else "U8"), [nb[k]]
                tensors.append((piece_name(fmt, prefix, L, e, k), dtype, shape, data))
            blobs[(L, e)] = b"".join(parts)
    return tensors, blobs


def dense_tensors(fmt, H, prefix):
    """A few non-expert tensors like the reference fixtures carry."""
    if fmt == 4:
        return [(prefix + "embed_tokens.weight", "BF16", [32, H], bytes(32 * H * 2)),
                (prefix + "norm.weight", "F32", [H], bytes(H * 4))]
    return [(prefix + "model.embed_tokens.weight", "BF16", [32, H], bytes(32 * H * 2)),
            (prefix + "model.layers.0.input_layernorm.weight", "BF16", [H], bytes(H * 2))]


def make_container(dirpath, rng, fmt, D, I, layers, n_experts, prefix="", n_files=1,
                   code_dtype="U8"):
    """Writes the experts (and a few dense tensors) over n_files files named like a
    sharded checkpoint; returns the expected blobs."""
    os.makedirs(dirpath, exist_ok=True)
    tensors, blobs = expert_tensors(rng, fmt, D, I, layers, n_experts, prefix, code_dtype)
    tensors = dense_tensors(fmt, D, prefix) + tensors
    per = (len(tensors) + n_files - 1) // n_files
    for i in range(n_files):
        part = tensors[i * per:(i + 1) * per]
        name = "model.safetensors" if n_files == 1 else \
            f"model-{i + 1:05d}-of-{n_files:05d}.safetensors"
        write_st(os.path.join(dirpath, name), part)
    return blobs

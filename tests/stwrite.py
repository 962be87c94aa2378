"""Writes safetensors files for the checkpoint tests, the way the reference's
tests build theirs (safetensors/safetensors_test.go:23-101): tensors laid out
contiguously, a header map the caller may mutate before it is written, and an
optional length prefix that lies."""
import json
import os
import struct

import numpy as np

SIZES = {"F64": 8, "F32": 4, "F16": 2, "BF16": 2, "I64": 8, "I32": 4, "I16": 2, "I8": 1,
         "U8": 1, "BOOL": 1}


def build(*tensors):
    """tensors: (name, dtype, shape, fill byte or bytes). -> (header dict, data bytes)."""
    hdr, data = {}, bytearray()
    for name, dtype, shape, fill in tensors:
        n = int(np.prod(shape)) if len(shape) else 1
        size = n * SIZES[dtype]
        begin = len(data)
        if isinstance(fill, (bytes, bytearray)):
            assert len(fill) == size
            data += fill
        else:
            data += bytes([fill]) * size
        hdr[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [begin, begin + size]}
    return hdr, bytes(data)


def good():
    """The file every refusal case starts from (safetensors_test.go:58-66)."""
    hdr, data = build(("a", "F32", [2, 2], 0x11), ("b", "BF16", [3], 0x22))
    hdr["__metadata__"] = {"format": "pt"}
    return hdr, data


def write_raw(path, js, data, length=None):
    n = len(js) if length is None else length
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", n))
        f.write(js)
        f.write(data)
    return path


def write(path, hdr, data, length=None):
    js = json.dumps(hdr, separators=(",", ":"), sort_keys=True).encode()
    return write_raw(path, js, data, length)


def write_arrays(path, arrays):
    """arrays: {name: (dtype, np array of the stored bits/values)} in a real file's layout."""
    tensors = []
    for name, (dtype, a) in sorted(arrays.items()):
        tensors.append((name, dtype, list(a.shape), np.ascontiguousarray(a).tobytes()))
    hdr, data = build(*tensors)
    js = json.dumps(hdr, separators=(",", ":"), sort_keys=True).encode()
    while (8 + len(js)) % 8:  # the reference writer pads the header with spaces
        js += b" "
    return write_raw(path, js, data)


def bf16_bits(x):
    """Top 16 bits of f32 (truncation; any bf16 pattern is a valid test input)."""
    return (np.asarray(x, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def write_index(dirpath, weight_map):
    with open(os.path.join(dirpath, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {"total_size": 22}, "weight_map": weight_map}, f)

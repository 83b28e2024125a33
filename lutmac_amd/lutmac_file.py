""".lutmac files with plane records (version 2), the producer side's file form.

Version 1 (the reference's src/format.cpp:146-290) stores every quantized
tensor as 256-weight AoS blocks with one scale each, so per-128-group scales
and RRQ-3 have no file form.  Version 2 keeps the same container -- magic
"LUTMAC01", u32 version, u32 metadata size, JSON metadata {"config",
"tensors"}, data from the next 256-byte boundary -- and adds a tensor record

    {"name", "shape": [rows, cols], "type": "planes", "format": "ternary" |
     "binary" | "rrq2" | "rrq3" | "int3" | "int4" | "int8", "group": G,
     "rotated": bool, "offset", "planes_bytes", "scales_bytes"}

whose data is the canonical planes [P][rows][cols/8] followed by the scales
[S][rows][groups] fp32 (lmx_planes_desc).  Raw fp32 tensors (norms, biases)
are {"name", "shape", "type": "raw", "offset"} as in version 1.  lmx_model_load
reads both versions; ``write`` produces version 2 from lmx_quantize output.
"""
import json
import struct

import numpy as np

from . import FMT_BINARY, FMT_INT3, FMT_INT4, FMT_INT8, FMT_RRQ2, FMT_RRQ3, FMT_TERNARY

FORMAT_KEYS = {FMT_TERNARY: "ternary", FMT_BINARY: "binary", FMT_RRQ2: "rrq2", FMT_RRQ3: "rrq3",
               FMT_INT3: "int3", FMT_INT4: "int4", FMT_INT8: "int8"}
ROTATED = {FMT_TERNARY, FMT_BINARY, FMT_RRQ2, FMT_RRQ3}   # lut_linear rotates these formats' activations


class Planes:
    """A quantized tensor in plane form: lmx_quantize's (planes, scales, group)
    for format fmt, rotated when the weights were FWHT-rotated first."""

    def __init__(self, fmt, planes, scales, group, rotated):
        self.fmt, self.group, self.rotated = fmt, int(group), bool(rotated)
        self.planes = np.ascontiguousarray(planes, np.uint8)
        self.scales = np.ascontiguousarray(scales, np.float32)

    @property
    def shape(self):
        return [int(self.planes.shape[1]), int(self.planes.shape[2] * 8)]


def write(path, config, tensors):
    """Write a version-2 .lutmac file.  config: the JSON config object (the
    reference's keys: vocab_size, hidden_size, intermediate_size,
    num_hidden_layers, num_attention_heads, num_key_value_heads, head_dim,
    rms_norm_eps, rope_theta, rope_scaling_factor, ...); tensors: a list of
    (name, Planes or a float32 array)."""
    records, blobs, off = [], [], 0
    for name, t in tensors:
        if isinstance(t, Planes):
            pb, sb = t.planes.tobytes(), t.scales.tobytes()
            records.append({"name": name, "shape": t.shape, "type": "planes", "format": FORMAT_KEYS[t.fmt],
                            "group": t.group, "rotated": t.rotated, "offset": off, "planes_bytes": len(pb),
                            "scales_bytes": len(sb)})
            data = pb + sb
        else:
            a = np.ascontiguousarray(t, np.float32)
            records.append({"name": name, "shape": list(a.shape), "type": "raw", "offset": off})
            data = a.tobytes()
        pad = (-len(data)) % 256
        blobs.append(data + b"\0" * pad)
        off += len(data) + pad
    meta = json.dumps({"config": config, "tensors": records}).encode()
    head = b"LUTMAC01" + struct.pack("<II", 2, len(meta)) + meta
    head += b"\0" * ((-len(head)) % 256)
    with open(path, "wb") as f:
        f.write(head)
        for b in blobs:
            f.write(b)

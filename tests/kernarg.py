"""kernarg.py -- the kernel-argument segments of the kernels in libexl3c4.so, read from the library's own code objects.

The radiance engine dispatches a kernel only if its argument segment (the explicit arguments plus any hidden argument
HIP appends for a kernel that reads one: blockDim, gridDim, printf's buffer, ...) fits its 768-byte slot
(kernels/exl3r4d/exl3r4d_dev.h:5-6, tests/gpu/kernarg_check.sh). hipLaunchKernel has no such limit, so only the code
object's metadata shows it. This reads the .hip_fatbin section of the shared library, cuts it at each clang offload
bundle (one a HIP translation unit), takes the gfx950 code object out of each and has llvm-readelf print its metadata
notes: per kernel its name, .kernarg_segment_size and the value kinds of its arguments.
"""
from __future__ import annotations

import os
import re
import shutil
import struct
import subprocess
import tempfile

LLVM = os.environ.get("ROCM_LLVM", "/opt/rocm/llvm/bin")
MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"


def tools_present() -> bool:
    return all(shutil.which(t) or os.path.exists(t) for t in ("objcopy", os.path.join(LLVM, "llvm-readelf")))


def code_objects(so_path: str):
    """The amdgcn code objects (bytes) of every offload bundle in the library's .hip_fatbin section."""
    with tempfile.TemporaryDirectory() as d:
        fb = os.path.join(d, "fb.bin")
        subprocess.run(["objcopy", "-O", "binary", "--only-section=.hip_fatbin", so_path, fb], check=True)
        data = open(fb, "rb").read()
    out = []
    for at in [m.start() for m in re.finditer(re.escape(MAGIC), data)]:
        n = struct.unpack_from("<Q", data, at + len(MAGIC))[0]
        q = at + len(MAGIC) + 8
        for _ in range(n):
            off, size, tl = struct.unpack_from("<QQQ", data, q)
            q += 24
            triple = data[q:q + tl].decode()
            q += tl
            if "amdgcn" in triple:
                out.append((triple, data[at + off:at + off + size]))
    return out


def kernels(so_path: str):
    """[{name, kernarg, hidden: [value kinds], by_value: [sizes]}] over every kernel of every code object."""
    res = []
    for _, co in code_objects(so_path):
        with tempfile.NamedTemporaryFile(suffix=".co") as f:
            f.write(co)
            f.flush()
            text = subprocess.run([os.path.join(LLVM, "llvm-readelf"), "--notes", f.name], check=True,
                                  capture_output=True, text=True).stdout
        # one kernel a list item of amdhsa.kernels, each starting "  - .agpr_count" (keys in sorted order)
        for item in re.split(r"\n  - (?=\.)", text.split("amdhsa.kernels:", 1)[1])[1:]:
            name = re.search(r"^\s*\.name:\s*(\S+)", item, re.M)
            size = re.search(r"^\s*\.kernarg_segment_size:\s*(\d+)", item, re.M)
            kinds = re.findall(r"\.value_kind:\s*(\S+)", item)
            byval = [int(x) for x in re.findall(r"\.size:\s*(\d+)\s*\n\s*\.value_kind:\s*by_value", item)]
            if name and size:
                res.append({"name": name.group(1), "kernarg": int(size.group(1)),
                            "hidden": [k for k in kinds if k.startswith("hidden_")], "by_value": byval})
    return res

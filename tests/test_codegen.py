"""CPU tier: properties of the generated gfx950 code that no run can show
reliably.

The decode attention kernel hands partial results between workgroups inside
one launch: each chunk stores its partial with agent-scope stores, then
arrives on a per-kv-head counter, and the last arrival reads every partial.
The arrival must follow the acknowledgement of all of the workgroup's
partial stores, or the merging workgroup can read a partial that has not
landed.  That ordering is an s_waitcnt vmcnt(0) between the last partial
store (the sc1 stores) and the barrier before the counter's atomic add.
A race would show up only rarely, so this checks the assembly directly."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


def _device_asm(src, tmp_path):
    if not shutil.which(HIPCC) and not os.path.exists(HIPCC):
        pytest.skip("hipcc not available")
    out = tmp_path / "k.s"
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-fhip-fp32-correctly-rounded-divide-sqrt",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "--cuda-device-only", "-S",
           "-o", str(out), os.path.join(ROOT, "zeninfer_amd", "csrc", src)]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-2000:]
    return out.read_text()


def _functions(asm, pattern):
    """(name, body) of every kernel whose symbol matches pattern."""
    found = []
    for m in re.finditer(r"^(_Z\S*" + pattern + r"\S*):", asm, re.M):
        end = asm.find(".Lfunc_end", m.end())
        found.append((m.group(1), asm[m.end():end]))
    return found


def test_attention_arrival_follows_partial_stores(tmp_path):
    asm = _device_asm("zq_layer.hip", tmp_path)
    kernels = _functions(asm, "attention_decode_kernel")
    assert kernels, "no attention_decode_kernel instantiation in the assembly"
    for name, body in kernels:
        lines = body.splitlines()
        atom = [i for i, l in enumerate(lines) if re.search(r"\bglobal_atomic_add\b", l)]
        assert len(atom) == 1, f"{name}: expected one counter atomic, found {len(atom)}"
        stores = [i for i, l in enumerate(lines[:atom[0]]) if re.search(r"\bglobal_store\w*\b.*\bsc1\b", l)]
        assert stores, f"{name}: no agent-scope partial stores before the counter"
        between = lines[stores[-1] + 1:atom[0]]
        wait = [i for i, l in enumerate(between) if re.search(r"s_waitcnt\s+vmcnt\(0\)", l)]
        barrier = [i for i, l in enumerate(between) if re.search(r"\bs_barrier\b", l)]
        assert wait and barrier and wait[0] < barrier[-1], (
            f"{name}: no s_waitcnt vmcnt(0) before the barrier between the last partial store and the counter")

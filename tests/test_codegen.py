"""CPU tier: properties of the generated gfx950 code that no run can show
reliably.

The decode attention kernel hands partial results between workgroups inside
one launch: each chunk stores its partial with agent-scope stores, then
arrives on a per-kv-head counter, and the last arrival reads every partial.
The arrival must follow the acknowledgement of all of the workgroup's
partial stores, or the merging workgroup can read a partial that has not
landed.  That ordering is an s_waitcnt vmcnt(0) between the last partial
store (the sc1 stores) and the barrier before the counter's atomic add.
A race would show up only rarely, so this checks the assembly directly.

Two build rules are checked the same way over every HIP source: no packed
fp32 arithmetic (the build disables the packed-fp32-ops feature; some forms
have given wrong results on these parts), and no writes through the scalar
data cache (stores, atomics, write-back or discard), which this code never
needs."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


SOURCES = ["zq_backend.hip", "zq_gemv.hip", "zq_gemm.hip", "zq_misc.hip", "zq_layer.hip", "zq_model.hip"]


@pytest.fixture(scope="module")
def device_asm(tmp_path_factory):
    """gfx950 assembly of every HIP source, with the library's own flags."""
    if not shutil.which(HIPCC) and not os.path.exists(HIPCC):
        pytest.skip("hipcc not available")
    from concurrent.futures import ThreadPoolExecutor
    from zeninfer_amd.build import FLAGS
    tmp = tmp_path_factory.mktemp("asm")
    flags = [f for f in FLAGS if f not in ("-shared", "-fPIC")]

    def one(src):
        out = tmp / (src + ".s")
        cmd = [HIPCC, *flags, "--cuda-device-only", "-S", "-o", str(out), os.path.join(ROOT, "zeninfer_amd", "csrc", src)]
        r = subprocess.run(cmd, capture_output=True, text=True, timeout=900)
        assert r.returncode == 0, r.stderr[-2000:]
        return src, out.read_text()

    with ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 1)) as ex:
        return dict(ex.map(one, SOURCES))


def _functions(asm, pattern):
    """(name, body) of every kernel whose symbol matches pattern."""
    found = []
    for m in re.finditer(r"^(_Z\S*" + pattern + r"\S*):", asm, re.M):
        end = asm.find(".Lfunc_end", m.end())
        found.append((m.group(1), asm[m.end():end]))
    return found


def test_attention_arrival_follows_partial_stores(device_asm):
    kernels = _functions(device_asm["zq_layer.hip"], "attention_decode_kernel")
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


def test_no_packed_fp32_arithmetic(device_asm):
    for src, asm in device_asm.items():
        hits = re.findall(r"^\s*(v_pk_(?:fma|add|mul)_f32)\b", asm, re.M)
        assert not hits, f"{src}: packed fp32 instructions {sorted(set(hits))}"


def test_no_scalar_cache_writes(device_asm):
    for src, asm in device_asm.items():
        hits = re.findall(r"^\s*(s_(?:store|buffer_store|scratch_store|atomic|buffer_atomic)\w*|s_dcache_(?:wb|discard)\w*)\b",
                          asm, re.M)
        assert not hits, f"{src}: scalar-cache writes {sorted(set(hits))}"


def test_no_kernel_spills_to_scratch(device_asm):
    """Every kernel of the library runs without private (scratch) memory:
    register spills on these streaming kernels cost more than any variant
    that needs them was worth (a Q4_0 GEMV step of four row groups spilled
    and was never run; a 64-K stage of the super-block GEMM spilled and was
    slower), so a change that makes one spill fails here before any run.
    Exempt: the int8 GEMMs' DOTS = true instantiations, the bit-exact test
    hook that stores every block's integer dot instead of accumulating; no
    product path launches them."""
    dots_mode = re.compile(r"gemm_i8_\w*kernelILi\d+ELb1E")
    bad, exempt = [], 0
    for src, asm in device_asm.items():
        for m in re.finditer(r"^\s*\.amdhsa_kernel (\S+)(.*?)\.end_amdhsa_kernel", asm, re.M | re.S):
            size = re.search(r"\.amdhsa_private_segment_fixed_size (\d+)", m.group(2))
            if size and int(size.group(1)) != 0:
                if dots_mode.search(m.group(1)):
                    exempt += 1
                else:
                    bad.append((src, m.group(1)[:120], int(size.group(1))))
    assert not bad, bad
    assert exempt <= 4  # today: the Q8_0 direct and tiled DOTS kernels

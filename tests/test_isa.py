"""The machine code of the hot kernels, on the CPU (hipcc cross-compiles for
gfx950): properties that the tests on the GPU see only as lost speed.

- Every K/V load of the decode stream takes a scalar buffer descriptor. A
  value the compiler takes for divergent in the address (once, a range bound
  that went through a cross-lane max) turns each load into a loop over the
  lanes (readfirstlane / compare / exec mask per load), which cost the e4m3
  decode 16% of its step.
- No kernel of the path spills registers to scratch memory or keeps a
  private stack.
"""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "optimize_inference_gpt-oss_amd", "csrc")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


def device_asm(tmp_path, name):
    out = tmp_path / (name + ".s")
    cmd = [HIPCC, "-std=c++17", "-O3", "-I", os.path.join(ROOT, "include"), "-I", CSRC, "-x",
           "hip", "--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "--cuda-device-only", "-S", os.path.join(CSRC, name + ".hip"),
           "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True, timeout=600)
    return out.read_text()


def kernels(asm, prefix):
    names = re.findall(r"^(_ZN3gkv\d+" + prefix + r"\w*):", asm, re.M)
    assert names, prefix
    for n in names:
        i = asm.index(n + ":")
        j = asm.index(".Lfunc_end", i)
        meta = asm[asm.index(".name:           " + n):]
        meta = meta[:meta.index(".vgpr_spill_count") + 40]
        yield n, asm[i:j], meta


def no_spills(meta, n):
    assert re.search(r"\.private_segment_fixed_size: 0\b", meta), n
    assert re.search(r"\.vgpr_spill_count: 0\b", meta), n


@pytest.mark.timeout(600)
def test_decode_stream_loads_take_scalar_descriptors(tmp_path):
    asm = device_asm(tmp_path, "decode_attention")
    for prefix in ("decode_fused_kernel", "decode_split_kernel"):
        for n, body, meta in kernels(asm, prefix):
            lines = body.splitlines()
            loads = [k for k, l in enumerate(lines) if "buffer_load_dwordx4" in l]
            assert loads, n
            for k in loads:
                before = " ".join(lines[max(0, k - 3):k])
                assert "s_and_saveexec" not in before, f"{n}: a load in a loop over lanes"
            no_spills(meta, n)


@pytest.mark.timeout(600)
def test_prefill_and_append_kernels_do_not_spill(tmp_path):
    """The prefill variants for groups of 4 to 8 query heads per kv head (gpt-oss
    has 8); those for 1 or 2 with a history keep a private stack (correct, slower,
    not on this path's shapes) and are not held to it."""
    for src, prefix in (("prefill_attention", r"prefill_kernelILi[48]E"),
                        ("kv_append", "kv_append_kernel"), ("qkv_append", "qkv_append_kernel")):
        asm = device_asm(tmp_path, src)
        for n, _, meta in kernels(asm, prefix):
            no_spills(meta, n)


@pytest.mark.timeout(600)
def test_direct_to_lds_scalar_bases_are_not_sign_extended(tmp_path):
    """The history prefill's direct-to-LDS loads take a wave-uniform 64-bit base
    in an SGPR pair (dma16_s). Its two halves are read from lane 0 with
    v_readfirstlane, whose result the compiler types as a signed int: widened
    as signed, a low half >= 2^31 would fill the high half with ones (a GPU
    memory fault, seen once when the allocator happened to hand out such an
    address). The high register of every such pair must be written by a
    readfirstlane (or a move), never by a sign extension of the low half."""
    asm = device_asm(tmp_path, "prefill_attention")
    n_loads = 0
    for n, body, _ in kernels(asm, r"prefill_kernel"):
        lines = body.splitlines()
        for k, l in enumerate(lines):
            m = re.search(r"global_load_lds_dwordx4 v\d+, s\[(\d+):(\d+)\]", l)
            if not m:
                continue
            n_loads += 1
            hi = "s" + m.group(2)
            # the last instruction before the load that writes the high register
            for d in reversed(lines[max(0, k - 200):k]):
                d = d.strip()
                if re.match(r"(s_|v_)\w+ " + hi + r"\b", d) or re.match(
                        r"(s_|v_)\w+ s\[(\d+):(\d+)\]", d) and hi in _pair_regs(d):
                    assert re.match(r"(v_readfirstlane_b32|s_mov_b32|s_mov_b64) ", d), \
                        f"{n}: high half {hi} of a direct-to-LDS base written by: {d}"
                    break
            assert not re.search(r"s_bfe_i64|s_ashr_i64", body), n
    assert n_loads > 0


def _pair_regs(line):
    m = re.match(r"(s_|v_)\w+ s\[(\d+):(\d+)\]", line.strip())
    return {"s" + str(i) for i in range(int(m.group(2)), int(m.group(3)) + 1)}

"""Properties of the gfx950 code the kernels compile to (CPU only: hipcc
cross-compiles). These guard numerics and safety properties that a test on
the GPU would only catch by chance:

* no fp16-result mixed-precision fma (v_fma_mixlo/hi_f16): the state must be
  narrowed from its rounded fp32 value, as the reference's StateIO does; a
  fused single rounding differs in rare ties and the compiler picks it per
  call site, which broke decode == prefill bit-identity for fp16 pools;
* no packed-fp32 VALU ops (v_pk_add/mul/fma_f32), which the build disables;
* no scalar-memory stores or atomics.
"""
from __future__ import annotations

import re
import shutil
import subprocess

import pytest

from braid_amd import build as B

SOURCES = ["gdn_scan.hip", "conv1d_decode.hip", "quant_act.hip", "gated_norm.hip", "hbm_probe.hip"]


@pytest.fixture(scope="module")
def asm(tmp_path_factory):
    hipcc = B.hipcc()
    if not shutil.which(hipcc) and not __import__("os").path.exists(hipcc):
        pytest.skip("hipcc not available")
    out = {}
    d = tmp_path_factory.mktemp("asm")
    for src in SOURCES:
        s = d / (src + ".s")
        cmd = [hipcc, *B.common_flags(), "-x", "hip", "--cuda-device-only", "-S",
               str(B.CSRC / src), "-o", str(s)]
        subprocess.run(cmd, check=True, capture_output=True)
        out[src] = s.read_text()
    return out


def _instructions(text):
    return [ln.split()[0] for ln in text.splitlines()
            if ln.strip() and ln.startswith((" ", "\t")) and not ln.strip().startswith((".", ";"))]


@pytest.mark.parametrize("src", SOURCES)
def test_no_fused_fp16_narrowing(asm, src):
    assert not re.search(r"v_(fma|mad)_mix(lo|hi)_f16", asm[src])


@pytest.mark.parametrize("src", SOURCES)
def test_no_packed_fp32_ops(asm, src):
    assert not re.search(r"\bv_pk_(add|mul|fma)_f32\b", asm[src])


@pytest.mark.parametrize("src", SOURCES)
def test_no_scalar_memory_writes(asm, src):
    ops = set(_instructions(asm[src]))
    bad = sorted(o for o in ops if re.match(r"s_(store|buffer_store|atomic|buffer_atomic|dcache_wb|dcache_discard)", o))
    assert not bad, bad


@pytest.mark.parametrize("src", SOURCES)
def test_no_kernel_spills_to_scratch(asm, src):
    """A spill in a bandwidth-bound kernel is extra memory traffic; the
    occupancy chosen for every kernel must fit its registers."""
    sizes = re.findall(r"\.amdhsa_private_segment_fixed_size\s+(\d+)", asm[src])
    assert sizes and all(int(x) == 0 for x in sizes), sizes


def test_decode_state_uses_128_bit_nontemporal_accesses(asm):
    text = asm["gdn_scan.hip"]
    assert re.search(r"global_load_dwordx4 .* nt", text)
    assert re.search(r"global_store_dwordx4 .* nt", text)


def test_decode_kernels_fit_four_waves_per_simd(asm):
    """The decode kernels are bound by the state stream, which needs four
    resident workgroups per CU (four waves per SIMD) to keep enough bytes in
    flight; that holds only at <= 128 architectural VGPRs per lane (except
    the instantiations for launches held to two workgroups per CU). Every
    instantiation (each pool dtype and gate policy, fused conv or not) is
    checked: the compiler's register count moves with small changes to the
    body's order."""
    text = asm["gdn_scan.hip"]
    found = []
    for m in re.finditer(r"\.amdhsa_kernel (\S+)(.*?)\.end_amdhsa_kernel", text, re.S):
        name, body = m.group(1), m.group(2)
        if "gdn_decode_kernel" not in name and "gdn_conv_decode_kernel" not in name:
            continue
        vgpr = int(re.search(r"\.amdhsa_next_free_vgpr\s+(\d+)", body).group(1))
        found.append((name, vgpr))
    # The instantiations for launches capped at two workgroups per CU
    # (kWavesPerSimd = 2, "ELi1ELi2E" in the mangled name) may use 256.
    capped = [(n, v) for n, v in found if "ELi1ELi2E" in n]
    assert len(capped) >= 6, len(capped)
    assert len(found) >= 9 + 24 + 6, len(found)
    over = [(n, v) for n, v in found if v > (256 if "ELi1ELi2E" in n else 128)]
    assert not over, over

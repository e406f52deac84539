"""Compiler resource report of the gfx950 kernels (CPU only: hipcc cross-compiles).

The attention kernels (matrix-core and exact-fp32), RoPE and the model
operators must not use scratch memory (register spills or run-time-indexed
private arrays), and the hot attention kernels must keep the occupancy their
tiling assumes.  The one documented exception is the causal combined backward
at head dims 16 and 32 for sequence lengths that are not a multiple of 64 (36
bytes per lane of spilled scalar registers).  At D = 64 every backward launch,
the separate dK/dV and dQ ones included, runs the combined kernel, which has
no scratch."""
import os
import re
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "gpt_from_scratch_amd", "csrc")
HIPCC = "/opt/rocm/bin/hipcc"
SOURCES = ("attn_fwd.hip", "attn_bwd.hip", "attn_valu.hip", "rope.hip", "model_ops.hip")
# the causal combined backward at head dims 16 and 32 for sequence lengths
# that are not a multiple of 64 (36 bytes per lane: scalar registers spilled)
ALLOWED_SCRATCH = re.compile(r"attn_bwd_kernel<mi::(BF16|F16), 64, true, (true|false), "
                             r"(16|32), true>")


def _hipflags(src):
    """HIPFLAGS of the library's Makefile, with the additions of src's object
    target, so the report is the shipped build's."""
    text = open(os.path.join(CSRC, "Makefile")).read()
    m = re.search(r"^HIPFLAGS = (.*?)(?<!\\)\n", text, re.S | re.M)
    flags = m.group(1).replace("\\\n", " ").replace("$(ARCH)", "gfx950").split()
    stem = src.rsplit(".", 1)[0]
    for extra in re.findall(r"^\$\(BUILD\)/" + re.escape(stem) + r"\.o: HIPFLAGS \+= (.*)$",
                            text, re.M):
        flags += extra.split()
    return [f for f in flags if f != "-fPIC"]


def _report(src, tmp):
    cmd = [HIPCC] + _hipflags(src) + ["-I" + os.path.join(ROOT, "include"), "--cuda-device-only",
                                   "-c", os.path.join(CSRC, src), "-o", os.path.join(tmp, src + ".o"),
                                   "-Rpass-analysis=kernel-resource-usage"]
    out = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert out.returncode == 0, out.stderr[-2000:]
    kernels = {}
    name = None
    for line in out.stderr.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            name = m.group(1)
            kernels[name] = {}
            continue
        m = re.search(r"remark:\s+(VGPRs|ScratchSize \[bytes/lane\]|Occupancy \[waves/SIMD\]): (\d+)", line)
        if m and name:
            kernels[name][m.group(1).split()[0]] = int(m.group(2))
    return kernels


@pytest.fixture(scope="module")
def reports(tmp_path_factory):
    if not os.path.exists(HIPCC):
        pytest.skip("hipcc not available")
    tmp = str(tmp_path_factory.mktemp("resources"))
    with ThreadPoolExecutor(len(SOURCES)) as ex:
        res = dict(zip(SOURCES, ex.map(lambda s: _report(s, tmp), SOURCES)))
    demangle = shutil.which("llvm-cxxfilt") or shutil.which("c++filt")
    if demangle is None:
        pytest.skip("no C++ demangler")
    names = [n for r in res.values() for n in r]
    pretty = subprocess.run([demangle], input="\n".join(names), capture_output=True, text=True).stdout
    mapping = dict(zip(names, pretty.splitlines()))
    return {src: {mapping.get(n, n): v for n, v in r.items()} for src, r in res.items()}


def test_no_scratch(reports):
    bad = []
    for src, kernels in reports.items():
        assert kernels, src
        for name, r in kernels.items():
            if r.get("ScratchSize", 0) and not ALLOWED_SCRATCH.search(name):
                bad.append((src, name, r["ScratchSize"]))
    assert not bad, bad


def test_attention_occupancy(reports):
    def find(src, pattern):
        hits = [(n, r) for n, r in reports[src].items() if re.search(pattern, n)]
        assert hits, pattern
        return hits

    # D = 64 forward: three workgroups of four waves per CU (the whole config-2 grid resident)
    for _, r in find("attn_fwd.hip", r"attn_fwd_mfma_kernel<mi::(BF16|F16), 64, "):
        assert r["Occupancy"] >= 3 and r["VGPRs"] <= 168
    # D = 128 forward and every backward launch: two waves per SIMD
    for _, r in find("attn_fwd.hip", r"attn_fwd_mfma_kernel<mi::(BF16|F16), 128, "):
        assert r["Occupancy"] >= 2
    for _, r in find("attn_bwd.hip", r"attn_bwd_kernel<mi::(BF16|F16), 64, "):
        assert r["Occupancy"] >= 2

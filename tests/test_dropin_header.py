"""The C++ drop-in header include/jhq_v14_streaming_add/jhq_gpu_index.cuh
against the reference's own caller: examples/demo_jhq_v14_streaming_add.cu
(unchanged, read where it lies in the reference checkout) must compile and link
with this repository's include/ directory ahead of the reference's, so that
"jhq_v14_streaming_add/jhq_gpu_index.cuh" resolves to the shim.  A small C++
program also exercises the shim's host-side behaviour without a GPU: the
constructor's argument checks throw std::invalid_argument with the reference's
messages (v14/jhq_gpu_index.cu:110-121), call-order errors throw
std::runtime_error."""
import os
import subprocess

import pytest

import jhq_gpu_amd as jg

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = "/root/reference"
DEMO = os.path.join(REF, "examples", "demo_jhq_v14_streaming_add.cu")
INC = os.path.join(ROOT, "include")
LIBDIR = os.path.dirname(jg.lib_path())


def _cxx(args, tmp_path):
    r = subprocess.run(["g++", "-std=c++17", "-O0"] + args, capture_output=True, text=True,
                       cwd=tmp_path)
    assert r.returncode == 0, r.stderr[-4000:]


@pytest.mark.skipif(not os.path.exists(DEMO), reason="reference checkout not present")
def test_reference_demo_compiles_and_links_unchanged(tmp_path):
    out = str(tmp_path / "demo_v14")
    _cxx(["-x", "c++", "-I", INC, "-I", REF, DEMO, "-x", "none", "-L", LIBDIR, "-ljhq_amd",
          "-Wl,-rpath," + LIBDIR, "-o", out], tmp_path)
    assert os.path.exists(out)


SHIM_PROBE = r'''
#include "jhq_v14_streaming_add/jhq_gpu_index.cuh"
#include <cstdio>
#include <cstring>
#include <vector>
int main() {
    jhq_gpu::JHQGpuIndex::Params p;
    if (p.M != 96 || p.B != 8 || p.Br != 4 || p.alpha != 4.0f || p.nlist != 1024 ||
        p.nprobe != 8 || p.ivf_iters != 8 || p.batch_size != 256 || p.seed != 42 ||
        p.add_batch != 65536) { std::puts("defaults"); return 1; }
    p.M = 3;
    try { jhq_gpu::JHQGpuIndex bad(10, p); std::puts("no throw"); return 1; }
    catch (const std::invalid_argument& e) {
        if (!std::strstr(e.what(), "divisible by M")) { std::puts(e.what()); return 1; }
    }
    p.M = 8; p.Br = 2;
    try { jhq_gpu::JHQGpuIndex bad(16, p); return 1; }
    catch (const std::invalid_argument& e) {
        if (!std::strstr(e.what(), "Br must be 4 or 8")) return 1;
    }
    p.Br = 4; p.nlist = 4; p.nprobe = 2;
    jhq_gpu::JHQGpuIndex ix(16, p);
    if (ix.dim() != 16 || ix.ntotal() != 0) return 1;
    std::vector<float> x(16 * 8, 0.5f);
    try { ix.add(x.data(), 8); return 1; }            // add before train
    catch (const std::runtime_error& e) {
        if (!std::strstr(e.what(), "train")) return 1;
    }
    std::vector<float> d(2 * 3); std::vector<int> l(2 * 3);
    try { ix.search(x.data(), 2, 3, d.data(), l.data()); return 1; }   // empty index
    catch (const std::runtime_error& e) {
        if (!std::strstr(e.what(), "empty")) return 1;
    }
    jhq_gpu::JHQGpuIndex moved(std::move(ix));
    std::puts("shim ok");
    return 0;
}
'''


def test_shim_host_behaviour(tmp_path):
    src = tmp_path / "probe.cpp"
    src.write_text(SHIM_PROBE)
    out = str(tmp_path / "probe")
    _cxx(["-I", INC, str(src), "-L", LIBDIR, "-ljhq_amd", "-Wl,-rpath," + LIBDIR, "-o", out],
         tmp_path)
    r = subprocess.run([out], capture_output=True, text=True)
    assert r.returncode == 0 and "shim ok" in r.stdout, (r.stdout, r.stderr)

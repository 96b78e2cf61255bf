"""The drop-in boundary links: the reference's own callers compile against the
host headers and link against liboracle_host / liborc_hip with no reference
implementation of the replaced files.

A maintainer keeps core/engine.cpp, core/tokenizer.cpp, core/machine_profile.cpp,
core/platform.cpp and bug/logger.cpp, and replaces core/{model,gguf_parser,
ops}.{hpp,cpp} (and core/sampler.* in the first configuration) with this
library's headers. Both configurations are checked: with this library's
Sampler, and with the reference's own core/sampler.cpp calling ops::argmax /
ops::softmax from this library. A third build uses this library's own
Engine and Tokenizer headers as well. The sources are read where they lie under
/root/reference through a symlink farm in a temporary directory; nothing is
copied into the repository and nothing built here ships. Skipped when the
reference tree is absent (the GPU box).
"""
import os
import shutil
import subprocess

import pytest

from conftest import ROOT as REPO

REF = "/root/reference"
HOST = os.path.join(REPO, "oracle-engine_amd", "host")
LIB = os.path.join(REPO, "oracle-engine_amd", "lib")
KEEP = ["core/engine.cpp", "core/engine.hpp", "core/tokenizer.cpp", "core/tokenizer.hpp",
        "core/machine_profile.cpp", "core/machine_profile.hpp", "core/platform.cpp", "core/platform.hpp",
        "bug/logger.cpp", "bug/logger.hpp"]
OURS = ["model.hpp", "gguf_parser.hpp", "gguf_types.hpp", "ops.hpp"]

MAIN = r'''
#include "core/engine.hpp"
#include "core/sampler.hpp"
#include "core/ops.hpp"
int main(int argc, char** argv) {
    Engine e;
    if (argc > 1) {  // never run by the test: the link is the check
        e.load(argv[1]);
        std::vector<Message> msgs{{"user", "hi"}};
        e.generate(msgs, GenParams{}, [](const std::string&) {});
        e.embed("hi");
        e.load_draft(argv[1]);
        Model m;
        m.load(argv[1]);
        auto snap = m.snapshot_kv(0);
        m.restore_kv(snap);
        int pos = 0;
        m.save_state("x.orkv", 0);
        m.load_state("x.orkv", pos);
        float v[4] = {1, 2, 3, 4};
        ops::softmax(v, 4);
        Sampler s(SamplerParams{}, 1);
        s.sample(v, 4);
        s.record(1);
        s.reset();
        s.set_params(SamplerParams{});
        (void)m.gguf().is_mmap_only();
    }
    return e.is_loaded() ? 0 : 1;
}
'''


def _farm(tmp, own_sampler):
    for d in ("core", "bug"):
        os.makedirs(os.path.join(tmp, d), exist_ok=True)
    keep = KEEP + ([] if own_sampler else ["core/sampler.cpp", "core/sampler.hpp"])
    for rel in keep:
        os.symlink(os.path.join(REF, rel), os.path.join(tmp, rel))
    for f in OURS + (["sampler.hpp"] if own_sampler else []):
        os.symlink(os.path.join(HOST, f), os.path.join(tmp, "core", f))
    with open(os.path.join(tmp, "main.cpp"), "w") as fh:
        fh.write(MAIN)
    return [r for r in keep if r.endswith(".cpp")] + ["main.cpp"]


def test_own_engine_headers_link(tmp_path):
    """The same caller program against this library's own Engine, Tokenizer,
    Sampler and ops headers (no reference file at all)."""
    assert os.path.exists(os.path.join(LIB, "liboracle_host.so")), "build the host library first"
    core = tmp_path / "core"
    core.mkdir()
    for f in OURS + ["sampler.hpp", "engine.hpp", "tokenizer.hpp", "spec.hpp"]:
        os.symlink(os.path.join(HOST, f), core / f)
    (tmp_path / "main.cpp").write_text(MAIN)
    exe = tmp_path / "engine_link"
    r = subprocess.run(["g++", "-std=c++17", "-O0", "-I", str(tmp_path), "-I", str(core), "-I",
                        os.path.join(REPO, "include"), str(tmp_path / "main.cpp"), "-o", str(exe), "-L", LIB,
                        "-loracle_host", "-lorc_hip", f"-Wl,-rpath,{LIB}", "-Wl,--no-undefined"],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]


@pytest.mark.skipif(not os.path.isdir(os.path.join(REF, "core")), reason="reference tree not present")
@pytest.mark.skipif(shutil.which("g++") is None, reason="no g++")
@pytest.mark.parametrize("own_sampler", [True, False], ids=["device-sampler", "reference-sampler"])
def test_reference_callers_link_against_host_library(tmp_path, own_sampler):
    assert os.path.exists(os.path.join(LIB, "liboracle_host.so")), "build the host library first"
    srcs = _farm(str(tmp_path), own_sampler)
    inc = ["-I", str(tmp_path), "-I", os.path.join(str(tmp_path), "core"), "-I", os.path.join(REPO, "include")]
    objs = []
    for s in srcs:
        o = os.path.join(str(tmp_path), os.path.basename(s) + ".o")
        r = subprocess.run(["g++", "-std=c++17", "-O0", "-fopenmp", *inc, "-c", os.path.join(str(tmp_path), s),
                            "-o", o], capture_output=True, text=True)
        assert r.returncode == 0, f"{s}: {r.stderr[-2000:]}"
        objs.append(o)
    exe = os.path.join(str(tmp_path), "engine_link")
    r = subprocess.run(["g++", "-o", exe, *objs, "-fopenmp", "-L", LIB, "-loracle_host", "-lorc_hip",
                        f"-Wl,-rpath,{LIB}", "-Wl,--no-undefined"], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]

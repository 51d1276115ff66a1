"""The reference-side binding shown in INTEGRATION.md must compile against the header.

INTEGRATION.md §2 shows the pybind11 section a maintainer adds to the reference's
``nimbleml_native`` (native/src/module.cpp). This test takes that exact ``cpp`` block,
places it after the includes a module.cpp has, adds the ``PYBIND11_MODULE`` that calls
``register_hip``, and runs ``g++ -fsyntax-only`` against ``include/nimbleml_hip.h`` and
pybind11, so a signature change in the header (an argument added, a type changed) fails
here instead of in the reference's build. It also checks that the block binds every
device-pointer function of the reference's CUDA section (module.cpp:229-285) under the
same name and argument names."""
import os
import re
import shutil
import subprocess
import sysconfig

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

# The reference's device-pointer section (module.cpp:229-285): name → argument names.
REFERENCE_DEVICE_API = {
    "flash_sdpa_forward_device": ["q", "k", "v", "out", "m", "l", "bh", "seq", "dk", "scale"],
    "flash_sdpa_backward_device": ["grad_out", "q", "k", "v", "m", "l", "grad_q", "grad_k",
                                   "grad_v", "bh", "seq", "dk", "scale"],
    "rmsnorm_forward_device": ["x", "gamma", "out", "ms", "rms", "rows", "dim", "eps"],
    "rmsnorm_backward_device": ["grad", "x", "gamma", "ms", "rms", "grad_x", "grad_gamma", "rows",
                                "dim", "eps"],
}


def _snippet():
    text = open(os.path.join(REPO, "INTEGRATION.md"), encoding="utf-8").read()
    sec = text[text.index("## 2. Binding on the reference side"):
               text.index("## 3. Binding used in this repository")]
    blocks = re.findall(r"```cpp\n(.*?)```", sec, flags=re.S)
    assert len(blocks) == 1, "INTEGRATION.md §2 must hold exactly one cpp block"
    return blocks[0]


def test_binding_names_and_arguments_match_the_reference():
    defs = {}
    for chunk in _snippet().split("m.def(")[1:]:
        name = re.match(r'"(\w+)"', chunk).group(1)
        defs[name] = re.findall(r'py::arg\("(\w+)"\)', chunk)
    for name, args in REFERENCE_DEVICE_API.items():
        assert name in defs, f"{name} is not bound"
        assert defs[name][:len(args)] == args, (name, defs[name])


def test_binding_compiles_against_the_header(tmp_path):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    import pybind11

    src = tmp_path / "module_hip.cpp"
    src.write_text(
        "#define NIMBLEML_WITH_HIP 1\n"
        "#include <pybind11/pybind11.h>\n#include <pybind11/numpy.h>\n"
        "namespace py = pybind11;\n" + _snippet() +
        "\nPYBIND11_MODULE(nimbleml_native, m) {\n#if defined(NIMBLEML_WITH_HIP)\n"
        "  register_hip(m);\n#endif\n}\n")
    cmd = [gxx, "-std=c++17", "-fsyntax-only", "-Wall", "-Werror=return-type",
           "-I", os.path.join(REPO, "include"), "-I", pybind11.get_include(),
           "-I", sysconfig.get_paths()["include"], str(src)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]

"""The C ABI without a GPU: the built library loads, exports every entry point the headers
in include/ declare, reports its offload arch, and the ctypes mirrors in navi_amd.abi have
the sizes and field offsets a C compiler gives the header's structs. No compute call is made.
"""
import ctypes as C
import re
import subprocess
from pathlib import Path

import pytest

from navi_amd import abi

ROOT = Path(__file__).resolve().parent.parent
HEADERS = sorted((ROOT / "include").glob("*.h"))


def _declared():
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        text = re.sub(r"//[^\n]*", "", text)
        names |= set(re.findall(r"\b(navi_[a-z0-9_]+)\s*\(", text))
    return names


def test_headers_declare_entry_points():
    assert HEADERS, "include/*.h missing"
    assert len(_declared()) >= 20


def test_library_exports_every_declared_symbol():
    lib = abi.lib()
    missing = [n for n in sorted(_declared()) if not hasattr(lib, n)]
    assert not missing, missing
    assert set(abi.EXPORTS) == _declared()


def test_library_is_built_for_gfx950():
    assert abi.lib().navi_build_arch().decode() == "gfx950"


def test_no_cpu_fallback_symbols():
    """The library exports only the declared ABI: no host compute path is hidden behind it."""
    out = subprocess.run(["nm", "-D", "--defined-only", str(abi.LIB_PATH)], capture_output=True, text=True, check=True)
    exported = {l.split()[-1] for l in out.stdout.splitlines() if " T " in l}
    navi = {s for s in exported if s.startswith("navi_")}
    assert navi == _declared()


STRUCTS = {
    "navi_device_info": abi.DeviceInfo, "navi_xformer_params": abi.XformerParams, "navi_model_params": abi.ModelParams,
    "navi_tensor_ref": abi.TensorRef, "navi_kv_view": abi.KvView, "navi_sampling": abi.Sampling,
    "navi_frame_options": abi.FrameOptions, "navi_frame_result": abi.FrameResult, "navi_prompt": abi.Prompt,
    "navi_vocoder_params": abi.VocoderParams, "navi_synth_request": abi.SynthRequest,
    "navi_synth_stats": abi.SynthStats, "navi_speaker_params": abi.SpeakerParams,
}


def test_ctypes_layouts_match_the_header(tmp_path):
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "navi_amd.h"', "int main(void) {"]
    for cname, py in STRUCTS.items():
        lines.append(f'printf("{cname} sizeof %zu\\n", sizeof({cname}));')
        for f in py._fields_:
            lines.append(f'printf("{cname} {f[0]} %zu\\n", offsetof({cname}, {f[0]}));')
    lines.append("return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", str(ROOT / "include"), "-o", str(exe), str(src)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split("\n")
    got = {}
    for l in out:
        if l:
            s, f, v = l.split()
            got[(s, f)] = int(v)
    for cname, py in STRUCTS.items():
        assert got[(cname, "sizeof")] == C.sizeof(py), cname
        for f in py._fields_:
            assert got[(cname, f[0])] == getattr(py, f[0]).offset, (cname, f[0])


def test_header_compiles_as_c_and_cpp(tmp_path):
    for lang, comp in (("c", "gcc"), ("c++", "g++")):
        src = tmp_path / f"inc.{'c' if lang == 'c' else 'cpp'}"
        src.write_text('#include "navi_amd.h"\nint main(void) { return NAVI_OK; }\n')
        subprocess.run([comp, "-Wall", "-Werror", "-I", str(ROOT / "include"), "-o", str(tmp_path / f"a_{lang}"), str(src)],
                       check=True)


def test_graph_facade_compiles(tmp_path):
    """navi_graph.hpp (the reference's Graph signatures over the C ABI) is self-contained C++20."""
    import subprocess
    src = tmp_path / "g.cpp"
    src.write_text('#include "navi_graph.hpp"\n'
                   'int main() { navi::qwen3tts::SynthRequest r; r.ids = {1, 2, 3}; navi::qwen3tts::SynthStats s;\n'
                   '  return static_cast<int>(r.ids.size()) + s.n_frames + navi::qwen3tts::STREAM_BATCH; }\n')
    r = subprocess.run(["g++", "-std=c++20", "-Wall", "-Wextra", "-Werror", "-fsyntax-only", f"-I{ROOT / 'include'}",
                        f"-I{ROOT / 'navi-tts_amd' / 'csrc' / 'host'}", str(src)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr

"""CPU-side checks of the BitNet engine library (libac_bitnet_hip.so): it exports the C entry points
include/ac_bitnet_engine_hip.h declares and the C++ methods of ameva::core::AcBitNetEngine that llama_bitnet_core.cpp
calls (adapters/bitnet/src/core/ac_bitnet_engine.h), the ctypes mirror's struct layouts equal the header's (compiled
with gcc), and without a GPU creation fails with a message instead of crashing. No GPU call succeeds here."""
import ctypes
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "ameva_compute_amd", "libac_bitnet_hip.so")

C_ENTRIES = ("ac_bitnet_engine_create", "ac_bitnet_engine_configure", "ac_bitnet_engine_upload_layer",
             "ac_bitnet_engine_upload_output", "ac_bitnet_engine_eval_token", "ac_bitnet_engine_lm_head",
             "ac_bitnet_engine_last_error", "ac_bitnet_engine_destroy")
# the reference header's members (ac_bitnet_engine.h), demangled
CXX_METHODS = ("ameva::core::AcBitNetEngine::Initialize()",
               "ameva::core::AcBitNetEngine::Configure(ameva::core::BitNetGpuConfig const&)",
               "ameva::core::AcBitNetEngine::UploadLayer(unsigned int, ameva::core::BitNetGpuLayerHost const&)",
               "ameva::core::AcBitNetEngine::UploadOutput(float const*, unsigned short const*, unsigned int)",
               "ameva::core::AcBitNetEngine::EvalToken(unsigned int, float const*, float*, float*, unsigned int)",
               "ameva::core::AcBitNetEngine::LMHead(float const*, float*)",
               "ameva::core::AcBitNetEngine::HasLMHead() const",
               "ameva::core::AcBitNetEngine::DeviceName[abi:cxx11]() const",
               "ameva::core::AcBitNetEngine::WeightBytes() const",
               "ameva::core::AcBitNetEngine::LMHeadBytes() const",
               "ameva::core::AcBitNetEngine::KVCacheBytes() const",
               "ameva::core::AcBitNetError::AcBitNetError(std::__cxx11::basic_string<char, std::char_traits<char>, "
               "std::allocator<char> > const&, int)")


@pytest.fixture(scope="module")
def exported():
    if not os.path.exists(LIB):
        pytest.skip("libac_bitnet_hip.so not built")
    out = subprocess.run(["nm", "-D", "--defined-only", "-C", LIB], check=True, capture_output=True, text=True).stdout
    return {line.split(" ", 2)[2] for line in out.splitlines() if line.count(" ") >= 2}


def test_exports_c_entries_and_engine_methods(exported):
    missing = [n for n in C_ENTRIES + CXX_METHODS if n not in exported]
    assert not missing, missing
    assert any(n.startswith("ameva::core::AcBitNetEngine::AcBitNetEngine()") for n in exported)
    assert any(n.startswith("ameva::core::AcBitNetEngine::~AcBitNetEngine()") for n in exported)


def test_ctypes_mirror_matches_the_header(tmp_path):
    from ameva_compute_amd import bitnet_engine as be
    src = tmp_path / "lay.c"
    src.write_text('#include <stddef.h>\n#include <stdio.h>\n#include "ac_bitnet_engine_hip.h"\n'
                   'int main(void){printf("%zu %zu %zu %zu %zu\\n", sizeof(AcBitNetConfigC), sizeof(AcBitNetLayerC),'
                   ' offsetof(AcBitNetConfigC, relu2_ffn), offsetof(AcBitNetLayerC, scale_wq),'
                   ' offsetof(AcBitNetLayerC, scale_w_down)); return 0;}\n')
    exe = tmp_path / "lay"
    subprocess.run(["gcc", "-std=c11", "-Wall", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)],
                   check=True)
    got = [int(v) for v in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()]
    want = [ctypes.sizeof(be.ConfigC), ctypes.sizeof(be.LayerC), be.ConfigC.relu2_ffn.offset,
            be.LayerC.scale_wq.offset, be.LayerC.scale_w_down.offset]
    assert got == want


def test_create_without_gpu_fails_with_a_message():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    from ameva_compute_amd import bitnet_engine as be
    with pytest.raises(be.AcBitNetError) as e:
        be.BitNetEngine()
    assert str(e.value)
    L = be.lib()
    assert L.ac_bitnet_engine_configure(None, None) != 0
    assert L.ac_bitnet_engine_eval_token(None, 0, None, None, None, 0) != 0
    L.ac_bitnet_engine_destroy(None)

"""The plugin's ggml layout (ameva_compute_amd/csrc/ggml_abi.h) against the ggml headers the reference vendors
(include/ggml/ggml.h, ggml-backend.h, ggml-backend-impl.h, and the ggml_cgraph / ggml_hash_set declarations of
ggml-impl.h): one C probe prints the size and every member offset of each struct and vtable the plugin fills or reads,
every enum value ggml_abi.h declares and the limits, compiled once against each header set; the two outputs must be
equal line for line. A header set that gave a vtable one more member, another GGML_MAX_NAME or a renumbered op fails
here. CPU only; skipped where /root/reference is absent (the GPU box).

ggml-impl.h includes gguf.h, which the reference does not vendor, so the two graph structs (and the bitset typedef
of the hash set) are read out of ggml-impl.h's text and compiled after ggml.h (the probe takes nothing else from that
header)."""
from __future__ import annotations

import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_INC = "/root/reference/include/ggml"
ABI_H = os.path.join(ROOT, "ameva_compute_amd", "csrc", "ggml_abi.h")

pytestmark = pytest.mark.skipif(not os.path.isdir(REF_INC), reason="the reference's ggml headers are absent")

STRUCTS = {
    "ggml_tensor": ["type", "buffer", "ne", "nb", "op", "op_params", "flags", "src", "view_src", "view_offs", "data",
                    "name", "extra"],
    "ggml_hash_set": ["size", "used", "keys"],
    "ggml_cgraph": ["size", "n_nodes", "n_leafs", "nodes", "grads", "grad_accs", "leafs", "use_counts",
                    "visited_hash_set", "order", "uid"],
    "ggml_backend_buffer_type_i": ["get_name", "alloc_buffer", "get_alignment", "get_max_size", "get_alloc_size",
                                   "is_host"],
    "ggml_backend_buffer_type": ["iface", "device", "context"],
    "ggml_backend_buffer_i": ["free_buffer", "get_base", "init_tensor", "memset_tensor", "set_tensor", "get_tensor",
                              "set_tensor_2d", "get_tensor_2d", "cpy_tensor", "clear", "reset"],
    "ggml_backend_buffer": ["iface", "buft", "context", "size", "usage"],
    "ggml_backend_i": ["get_name", "free", "set_tensor_async", "get_tensor_async", "set_tensor_2d_async",
                       "get_tensor_2d_async", "cpy_tensor_async", "synchronize", "graph_plan_create",
                       "graph_plan_free", "graph_plan_update", "graph_plan_compute", "graph_compute", "event_record",
                       "event_wait", "graph_optimize"],
    "ggml_backend": ["guid", "iface", "device", "context"],
    "ggml_backend_device_i": ["get_name", "get_description", "get_memory", "get_type", "get_props", "init_backend",
                              "get_buffer_type", "get_host_buffer_type", "buffer_from_host_ptr", "supports_op",
                              "supports_buft", "offload_op", "event_new", "event_free", "event_synchronize"],
    "ggml_backend_device": ["iface", "reg", "context"],
    "ggml_backend_reg_i": ["get_name", "get_device_count", "get_device", "get_proc_address"],
    "ggml_backend_reg": ["api_version", "iface", "context"],
    "ggml_backend_dev_caps": ["async", "host_buffer", "buffer_from_host_ptr", "events"],
    "ggml_backend_dev_props": ["name", "description", "memory_free", "memory_total", "type", "device_id", "caps"],
}
MACROS = ["GGML_MAX_DIMS", "GGML_MAX_OP_PARAMS", "GGML_MAX_SRC", "GGML_MAX_NAME", "GGML_BACKEND_API_VERSION"]


def _enum_names() -> list[str]:
    text = open(ABI_H).read()
    names = re.findall(r"\b(GGML_(?:TYPE|OP|GLU_OP|STATUS|BACKEND_BUFFER_USAGE|BACKEND_DEVICE_TYPE)_[A-Z0-9_]+)\b",
                       text)
    return sorted(set(names))


def _probe_body() -> str:
    lines = []
    for s, members in STRUCTS.items():
        lines.append(f'printf("sizeof {s} %zu\\n", sizeof(struct {s}));')
        for m in members:
            lines.append(f'printf("offsetof {s}.{m} %zu\\n", offsetof(struct {s}, {m}));')
    for e in _enum_names():
        lines.append(f'printf("enum {e} %lld\\n", (long long){e});')
    for m in MACROS:
        lines.append(f'printf("macro {m} %lld\\n", (long long)({m}));')
    return "int main(void) {\n" + "\n".join("    " + x for x in lines) + "\n    return 0;\n}\n"


def _graph_structs_from_ref() -> str:
    text = open(os.path.join(REF_INC, "ggml-impl.h")).read()
    out = []
    for pat in (r"typedef uint32_t ggml_bitset_t;", r"struct ggml_hash_set \{.*?\};",
                r"enum ggml_cgraph_eval_order \{.*?\};", r"struct ggml_cgraph \{.*?\};"):
        m = re.search(pat, text, re.S)
        assert m, pat
        out.append(m.group(0))
    return "\n".join(out)


def _run(tmp_path, name: str, prologue: str, flags: list[str]) -> list[str]:
    src = tmp_path / f"{name}.c"
    exe = tmp_path / name
    src.write_text("#include <stddef.h>\n#include <stdio.h>\n" + prologue + "\n" + _probe_body())
    r = subprocess.run(["gcc", "-std=gnu11", "-w", *flags, "-o", str(exe), str(src)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]
    return subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.splitlines()


def test_ggml_abi_h_matches_the_reference_headers(tmp_path):
    ref = _run(tmp_path, "probe_ref", '#include "ggml.h"\n#include "ggml-backend.h"\n#include "ggml-backend-impl.h"\n'
               + _graph_structs_from_ref(), ["-I" + REF_INC])
    ours = _run(tmp_path, "probe_ours", f'#include "{ABI_H}"', [])
    assert len(ref) == len(ours) > 150
    diff = [(a, b) for a, b in zip(ref, ours) if a != b]
    assert not diff, diff[:20]
    # the figures the plugin's static_asserts and its ctypes mirror in tests/ggml_plugin.py rely on
    d = dict(line.rsplit(" ", 1) for line in ours)
    assert d["sizeof ggml_tensor"] == "336" and d["offsetof ggml_tensor.data"] == "248"
    assert d["enum GGML_OP_FLASH_ATTN_EXT"] == "74" and d["enum GGML_OP_GLU"] == "96"
    assert d["enum GGML_OP_SET_ROWS"] == "42" and d["enum GGML_TYPE_Q4_K"] == "12"

"""The C-ABI library loads, exports every function include/uttt_amd.h declares, and the
ctypes structures match the C layout (checked against gcc's offsetof on the header).
No kernel is launched: only host-side calls that return before touching a GPU."""
import ctypes as C
import os
import re
import subprocess
import tempfile

import pytest

from utttcompanion_amd import _native as N
from utttcompanion_amd import build

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "uttt_amd.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(uttt_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(build.LIB_PATH):
        build.build()
    return N.load_library()


def test_every_declared_symbol_is_exported_and_typed(lib):
    names = declared_functions()
    assert len(names) >= 9
    for name in names:
        assert name in N.SIGNATURES, f"{name} has no ctypes signature"
        assert hasattr(lib, name), f"{name} not exported"
    assert set(N.SIGNATURES) == set(names)


def test_struct_layouts_match_the_c_header(tmp_path):
    structs = {"uttt_chunk_update_args": N.ChunkUpdateArgs, "uttt_readout_args": N.ReadoutArgs,
               "uttt_rope_append_args": N.RopeAppendArgs, "uttt_swa_prefill_args": N.SwaPrefillArgs,
               "uttt_swa_decode_args": N.SwaDecodeArgs, "uttt_elastic_pull_args": N.ElasticPullArgs,
               "uttt_chunk_chain_args": N.ChunkChainArgs, "uttt_proj_epilogue_args": N.ProjEpilogueArgs,
               "uttt_skinny_linear_args": N.SkinnyLinearArgs, "uttt_greedy_args": N.GreedyArgs,
               "uttt_layer_update_args": N.LayerUpdateArgs, "uttt_linear_args": N.LinearArgs,
               "uttt_prefill_layer_calls": N.PrefillLayerCalls, "uttt_prefill_chunk_args": N.PrefillChunkArgs}
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', 'int main(void) {']
    for cname, py in structs.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for field, _ in py._fields_:
            lines.append(f'printf("{cname} {field} %zu\\n", offsetof({cname}, {field}));')
    lines.append("return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-o", str(exe), str(src)], check=True)
    out = subprocess.run([str(exe)], check=True, stdout=subprocess.PIPE, text=True).stdout.split("\n")
    got = {}
    for line in out:
        if line:
            cname, field, value = line.split()
            got[(cname, field)] = int(value)
    for cname, py in structs.items():
        assert got[(cname, "size")] == C.sizeof(py), cname
        for field, _ in py._fields_:
            assert got[(cname, field)] == getattr(py, field).offset, f"{cname}.{field}"


def test_host_side_calls(lib):
    assert lib.uttt_abi_version() == N.ABI_VERSION
    ws = lib.uttt_chunk_update_workspace(8, 768, 2048, N.DTYPE_BF16)
    assert ws > 8 * 64 * 2048 * 4
    assert lib.uttt_chunk_update_workspace(8, 770, 2048, N.DTYPE_BF16) == 0  # invalid d_model
    assert lib.uttt_readout_workspace(2, 100, 512, 1024, N.DTYPE_F32) > 0
    assert lib.uttt_chunk_chain_workspace(8, 12, 768, 2048, N.DTYPE_BF16) > 12 * 8 * 64 * 2048 * 2 * 7
    assert lib.uttt_chunk_chain_workspace(8, N.MAX_CHAIN + 1, 768, 2048, N.DTYPE_BF16) == 0  # too many layers


def test_invalid_arguments_are_rejected_before_any_launch(lib):
    a = N.ChunkUpdateArgs()
    a.batch, a.tokens, a.d_model, a.d_ff = 1, 0, 512, 1024
    rc = lib.uttt_chunk_update(C.byref(a), None, 0, None)
    assert rc == 1
    assert b"tokens per chunk" in lib.uttt_last_error()
    p = N.SwaPrefillArgs()
    p.batch, p.n_heads, p.n_kv_heads, p.head_dim = 1, 4, 3, 64
    assert lib.uttt_swa_prefill(C.byref(p), None) == 1
    assert b"n_kv_heads" in lib.uttt_last_error()
    ch = N.ChunkChainArgs()
    ch.batch, ch.layers, ch.tokens, ch.d_model, ch.d_ff = 2, 3, 64, 512, 1024
    assert lib.uttt_chunk_chain(C.byref(ch), None, 0, None) == 1
    assert b"layer 0 must be non-NULL" in lib.uttt_last_error()
    ch.layers = 0
    assert lib.uttt_chunk_chain(C.byref(ch), None, 0, None) == 1
    assert b"layers must be in" in lib.uttt_last_error()
    d = N.SwaDecodeArgs()
    d.head_dim = 96
    assert lib.uttt_swa_decode(C.byref(d), None) == 1
    assert b"head_dim" in lib.uttt_last_error()
    s = N.SkinnyLinearArgs()
    s.m, s.n, s.k, s.act_dtype = 65, 64, 64, N.DTYPE_BF16
    assert lib.uttt_skinny_linear(C.byref(s), None) == 1
    assert b"m must be in" in lib.uttt_last_error()
    s.m, s.n = 8, 48
    assert lib.uttt_skinny_linear(C.byref(s), None) == 1
    assert b"multiple of 32" in lib.uttt_last_error()
    s.n, s.act_dtype = 64, N.DTYPE_F32
    assert lib.uttt_skinny_linear(C.byref(s), None) == 1
    assert b"bf16" in lib.uttt_last_error()


def test_prefill_chunk_refuses_missing_events_before_any_launch(lib):
    """The chunk executor keeps no state of its own: the events that order its two streams come
    from the caller, and a call without a full set is refused before anything is enqueued."""
    ch = N.ChunkChainArgs()
    ch.layers = 2
    calls = (N.PrefillLayerCalls * 2)()
    a = N.PrefillChunkArgs()
    a.n_layers, a.layers, a.chain = 2, C.cast(calls, C.POINTER(N.PrefillLayerCalls)), C.pointer(ch)
    assert lib.uttt_prefill_chunk(C.byref(a), C.c_void_p(1), C.c_void_p(2)) == 1
    assert b"caller-owned events" in lib.uttt_last_error()
    ev = (C.c_void_p * 5)(*([C.c_void_p(8)] * 5))
    a.events, a.n_events = C.cast(ev, C.POINTER(C.c_void_p)), 5  # 2 n_layers + 2 = 6 needed
    assert lib.uttt_prefill_chunk(C.byref(a), C.c_void_p(1), C.c_void_p(2)) == 1
    assert b"2 n_layers + 2 = 6" in lib.uttt_last_error()
    ev6 = (C.c_void_p * 6)(*([C.c_void_p(8)] * 5 + [None]))
    a.events, a.n_events = C.cast(ev6, C.POINTER(C.c_void_p)), 6
    assert lib.uttt_prefill_chunk(C.byref(a), C.c_void_p(1), C.c_void_p(2)) == 1
    assert b"events[5] is NULL" in lib.uttt_last_error()
    a.defer_join = 2
    assert lib.uttt_prefill_chunk(C.byref(a), C.c_void_p(1), C.c_void_p(2)) == 1
    assert b"defer_join must be 0 or 1" in lib.uttt_last_error()
    assert lib.uttt_events_create(1, None) == 1
    assert lib.uttt_events_destroy(1, None) == 1
    assert lib.uttt_stream_wait_event(None, None) == 1
    assert b"event must be non-NULL" in lib.uttt_last_error()

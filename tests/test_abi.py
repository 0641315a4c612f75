"""The C-ABI library loads and exports every function include/tlm_hip.h
declares, and the ctypes structure layouts equal the C compiler's (no GPU
compute calls here)."""
import ctypes as C
import os
import re
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HDR = os.path.join(ROOT, "include", "tlm_hip.h")


def declared_functions():
    src = open(HDR).read()
    src = re.sub(r"/\*.*?\*/", " ", src, flags=re.S)
    names = re.findall(r"\b(tlm_\w+)\s*\(", src)
    typedefs = set(re.findall(r"\(\*\s*(tlm_\w+)\)", src))
    return sorted(set(names) - typedefs)


def test_library_exports_every_declared_symbol():
    from tierlm_amd import lib
    out = subprocess.run(["nm", "-D", "--defined-only", lib._name], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r" T (\w+)$", out, flags=re.M))
    decl = declared_functions()
    assert len(decl) >= 20
    missing = [n for n in decl if n not in exported]
    assert not missing, missing


def test_python_binding_covers_header():
    from tierlm_amd import EXPORTS
    assert sorted(EXPORTS) == declared_functions()


def test_struct_layouts_match_c():
    from tierlm_amd._lib import (ExpertRef, ExpertSrc, ModelGeom, ModelSynthOpts, MoeDesc, PacketLoc, QuantKernels,
                                 Seg, StackOpts, StoreOpts, StoreStats, TensorRef)
    from tierlm_amd.model import ModelOpts, ModelStats
    prog = r'''
#include <stdio.h>
#include <stddef.h>
#include "tlm_hip.h"
#define O(T, f) printf(#T "." #f " %zu\n", offsetof(T, f))
int main(void) {
  printf("seg %zu\nmoe %zu\nqk %zu\n", sizeof(tlm_hip_seg), sizeof(tlm_hip_moe_desc), sizeof(tlm_hip_quant_kernels));
  O(tlm_hip_seg, W); O(tlm_hip_seg, row_bytes); O(tlm_hip_seg, act); O(tlm_hip_seg, y); O(tlm_hip_seg, rows);
  O(tlm_hip_moe_desc, E); O(tlm_hip_moe_desc, routed_scale); O(tlm_hip_moe_desc, expert_dt);
  O(tlm_hip_moe_desc, ffn_norm); O(tlm_hip_moe_desc, experts); O(tlm_hip_moe_desc, shared_gate_inp);
  O(tlm_hip_quant_kernels, dot); O(tlm_hip_quant_kernels, mv);
  printf("src %zu\nopts %zu\nref %zu\nstats %zu\n", sizeof(tlm_hip_expert_src), sizeof(tlm_hip_store_opts),
         sizeof(tlm_hip_expert_ref), sizeof(tlm_hip_store_stats));
  O(tlm_hip_expert_src, id); O(tlm_hip_expert_src, dtype); O(tlm_hip_expert_src, item_off);
  O(tlm_hip_expert_src, payload_len); O(tlm_hip_expert_src, payload);
  O(tlm_hip_store_opts, top_k); O(tlm_hip_store_opts, pin_frac); O(tlm_hip_store_opts, fetch);
  O(tlm_hip_store_opts, fetch_user); O(tlm_hip_expert_ref, mats);
  O(tlm_hip_store_stats, wait_ns); O(tlm_hip_store_stats, slots); O(tlm_hip_store_stats, in_use);
  printf("loc %zu\ngeom %zu\ntref %zu\n", sizeof(tlm_hip_packet_loc), sizeof(tlm_hip_model_geom),
         sizeof(tlm_hip_tensor_ref));
  O(tlm_hip_packet_loc, flags); O(tlm_hip_packet_loc, offset); O(tlm_hip_packet_loc, crc32c); O(tlm_hip_packet_loc, heat);
  O(tlm_hip_model_geom, router); O(tlm_hip_model_geom, rope_theta); O(tlm_hip_model_geom, rope_orig_len);
  O(tlm_hip_tensor_ref, dtype); O(tlm_hip_tensor_ref, shape); O(tlm_hip_tensor_ref, nbytes);
  printf("synth %zu\nmopts %zu\n", sizeof(tlm_hip_model_synth_opts), sizeof(tlm_hip_model_opts));
  O(tlm_hip_model_synth_opts, qk_norm); O(tlm_hip_model_synth_opts, seed); O(tlm_hip_model_synth_opts, heat_gamma);
  O(tlm_hip_model_opts, attn_split); O(tlm_hip_model_opts, expert_cache_bytes); O(tlm_hip_model_opts, pin_frac);
  O(tlm_hip_model_opts, lookahead_k); O(tlm_hip_model_opts, interest); O(tlm_hip_model_opts, prefill_chunk);
  O(tlm_hip_model_opts, stats); O(tlm_hip_model_opts, host_routes);
  printf("sopts %zu\n", sizeof(tlm_hip_stack_opts));
  O(tlm_hip_stack_opts, interest); O(tlm_hip_stack_opts, instinct_seen); O(tlm_hip_stack_opts, host_routes);
  printf("mstats %zu\n", sizeof(tlm_hip_model_stats));
  O(tlm_hip_model_stats, attn_ns); O(tlm_hip_model_stats, expert_wait_ns); O(tlm_hip_model_stats, other_ns);
  return 0;
}'''
    with tempfile.TemporaryDirectory() as d:
        c = os.path.join(d, "p.c")
        open(c, "w").write(prog)
        exe = os.path.join(d, "p")
        subprocess.run(["gcc", "-std=c11", "-I" + os.path.join(ROOT, "include"), c, "-o", exe], check=True)
        vals = dict(line.rsplit(" ", 1) for line in subprocess.run([exe], capture_output=True, text=True,
                                                                   check=True).stdout.splitlines())
    vals = {k: int(v) for k, v in vals.items()}
    assert vals["seg"] == C.sizeof(Seg)
    assert vals["moe"] == C.sizeof(MoeDesc)
    assert vals["qk"] == C.sizeof(QuantKernels)
    for name, cls in (("src", ExpertSrc), ("opts", StoreOpts), ("ref", ExpertRef), ("stats", StoreStats),
                      ("loc", PacketLoc), ("geom", ModelGeom), ("tref", TensorRef), ("synth", ModelSynthOpts),
                      ("mopts", ModelOpts), ("sopts", StackOpts), ("mstats", ModelStats)):
        assert vals[name] == C.sizeof(cls), name
    for k, v in vals.items():
        if "." not in k:
            continue
        t, f = k.split(".")
        cls = {"tlm_hip_seg": Seg, "tlm_hip_moe_desc": MoeDesc, "tlm_hip_quant_kernels": QuantKernels,
               "tlm_hip_expert_src": ExpertSrc, "tlm_hip_store_opts": StoreOpts, "tlm_hip_expert_ref": ExpertRef,
               "tlm_hip_store_stats": StoreStats, "tlm_hip_packet_loc": PacketLoc, "tlm_hip_model_geom": ModelGeom,
               "tlm_hip_tensor_ref": TensorRef, "tlm_hip_model_synth_opts": ModelSynthOpts,
               "tlm_hip_model_opts": ModelOpts, "tlm_hip_stack_opts": StackOpts,
               "tlm_hip_model_stats": ModelStats}[t]
        assert getattr(cls, f).offset == v, k


def test_tier_before_init_and_without_gpu():
    """Without a device the tier stays "none" and fill reports 0 entries."""
    import torch

    from tierlm_amd import lib, quant
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    assert quant.tier() == "none"
    k, got = quant.kernel_table()
    assert got == 0
    assert lib.tlm_hip_init(0) == -7          # TLM_EUNSUP: no HIP device
    assert b"no HIP device" in lib.tlm_hip_errmsg()


def test_host_checks_reject_bad_arguments_without_launching():
    """Argument validation happens on the host, before any launch."""
    from tierlm_amd import lib
    from tierlm_amd._lib import MoeDesc
    d = MoeDesc()
    d.E, d.k, d.D, d.de = 0, 8, 2048, 768
    assert lib.tlm_hip_moe_layer(C.byref(d), C.c_void_p(16), None, None, C.c_void_p(256), None) == -3
    assert lib.tlm_hip_moe_layer_phase(C.byref(d), 4, C.c_void_p(16), None, None, C.c_void_p(256), None) == -3
    assert lib.tlm_hip_packed_bytes(14, 768, 2048) == 768 * 8 * 210
    assert lib.tlm_hip_packed_bytes(14, 37, 256) == 48 * 210        # last tile padded to 16 rows
    assert lib.tlm_hip_packed_bytes(14, 16, 100) == 0
    assert lib.tlm_hip_qact_bytes(15, 257) == 584
    assert lib.tlm_hip_qact_bytes(8, 33) == 72
    assert lib.tlm_hip_quantize_act(15, None, 256, None, None) == -3
    assert lib.tlm_hip_quantize_act(15, None, 0, None, None) == 0     # n <= 0 is a no-op


def _device_symbols(so_bytes):
    """Global symbol names of every gfx950 code object in the library's
    offload bundles (format: magic, entry count, then per entry offset, size,
    triple length and triple; each entry an ELF64 code object)."""
    import struct
    magic = b"__CLANG_OFFLOAD_BUNDLE__"
    names, n_objs = set(), 0
    at = so_bytes.find(magic)
    while at >= 0:
        (n,) = struct.unpack_from("<Q", so_bytes, at + 24)
        p = at + 32
        for _ in range(n):
            off, size, tlen = struct.unpack_from("<QQQ", so_bytes, p)
            triple = so_bytes[p + 24:p + 24 + tlen].decode()
            p += 24 + tlen
            if "gfx950" not in triple:
                continue
            elf = so_bytes[at + off:at + off + size]
            assert elf[:4] == b"\x7fELF", triple
            n_objs += 1
            shoff, = struct.unpack_from("<Q", elf, 0x28)
            shentsize, shnum = struct.unpack_from("<HH", elf, 0x3A)
            secs = [struct.unpack_from("<IIQQQQIIQQ", elf, shoff + i * shentsize) for i in range(shnum)]
            for s in secs:
                if s[1] != 2:   # SHT_SYMTAB
                    continue
                strtab = secs[s[6]]
                for j in range(s[5] // 24):
                    st_name, st_info = struct.unpack_from("<IB", elf, s[4] + j * 24)
                    if st_info >> 4 != 1:   # STB_GLOBAL
                        continue
                    end = elf.index(b"\0", strtab[4] + st_name)
                    names.add(elf[strtab[4] + st_name:end].decode())
        at = so_bytes.find(magic, at + 24)
    return names, n_objs


def test_registered_kernels_exist_in_code_objects():
    """Every kernel and device variable the host code registers by name (the
    mangled names in .rodata) is a global symbol of one of the library's
    gfx950 code objects: the runtime looks kernels up by those names when it
    loads a module at its first launch, and a name that the host and device
    passes mangle differently fails that load."""
    import re
    so = os.path.join(ROOT, "tierlm_amd", "libtlm_hip.so")
    if not os.path.exists(so):
        pytest.skip("library not built")
    data = open(so, "rb").read()
    dev, n_objs = _device_symbols(data)
    assert n_objs >= 6, n_objs
    out = subprocess.run(["/opt/rocm/llvm/bin/llvm-readelf", "-p", ".rodata", so], capture_output=True, text=True,
                         check=True).stdout
    registered = {m.group(1) for m in re.finditer(r"\]\s+(_Z\S+)", out)}
    assert len(registered) > 100
    missing = sorted(registered - dev)
    assert not missing, missing[:5]

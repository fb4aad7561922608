"""Rules the built gfx950 code objects must keep (llvm-objdump of our own build).

1. Wait-state hazards of the hand-written MFMAs of the H = 128 kernels.
decode_h128.hip issues its MFMAs by inline asm (each must keep its slot of the
static schedule), so the compiler's hazard recognizer does not see them and
the kernel must provide their wait states itself.  This test reads the
gfx950 code object of the built decode_h128.o (llvm-objdump of our own
build) and checks, along every control-flow path (branch targets included):

* a VALU write of a VGPR that an MFMA reads (A, B, C or scale operand) is at
  least 2 wait states before the MFMA;
* an MFMA's result registers are neither read nor written by a VALU, LDS or
  memory instruction within 20 wait states after it (a VALU read of a 16-pass
  XDL result needs 19), except by the next MFMA of a same-shape accumulate
  chain on those registers.

s_nop N counts N + 1 wait states, every other instruction one.

2. Every LDS-DMA (global_load_lds_*) follows the last write of M0 by at least
one wait state (gfx9-family rule for an SALU write of M0 read by an LDS DMA).
3. No scalar-memory stores, atomics or cache write-backs in any kernel.
4. No packed-FP32 add/mul/fma (the build disables their formation).
5. No decode, combine, quant or planner kernel spills to scratch (code-object
   metadata: private segment size and VGPR spill count 0), except the a16w8
   variant of the 16-head kernel (two fp8 terms of Q, 80 registers, at two
   work-groups per CU), which is on no benchmarked route.

``python tests/test_isa_rules.py --resources`` prints the per-kernel register,
LDS and scratch figures of the built library as a markdown table.
"""
import os
import re
import subprocess
import sys
import tempfile

import pytest
import yaml

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BUILD = os.path.join(ROOT, "amd_optimization_challenge_amd", "_build")
OBJ = os.path.join(BUILD, "decode_h128.o")
LLVM = "/opt/rocm/llvm/bin"
PRE_WS, POST_WS = 2, 20

INSN = re.compile(r"^\s+(\S+)\s*(.*?)\s*//\s*([0-9A-Fa-f]+):(.*)$")
TARGET = re.compile(r"<(\S+?)(?:\+0x([0-9a-f]+))?>")
FUNC = re.compile(r"^([0-9a-f]+) <(\S+)>:$")
REG = re.compile(r"\b([va])(?:\[(\d+):(\d+)\]|(\d+)(?!\d))")


def regs(text):
    out = set()
    for m in REG.finditer(text):
        if m.group(4) is not None:
            out.add((m.group(1), int(m.group(4))))
        else:
            out |= {(m.group(1), i) for i in range(int(m.group(2)), int(m.group(3)) + 1)}
    return out


def operands(args):
    args = re.split(r"\s(?:op_sel|op_sel_hi|cbsz|abid|blgp|offset|glc|slc|nt|sc0|sc1)\b", args)[0]
    return [a.strip() for a in args.split(",") if a.strip()]


def disassemble(obj, tmp):
    fat = os.path.join(tmp, "fat.bin")
    co = os.path.join(tmp, "dev.co")
    subprocess.run([f"{LLVM}/llvm-objcopy", f"--dump-section=.hip_fatbin={fat}", obj, os.path.join(tmp, "host.o")],
                   check=True, capture_output=True)
    subprocess.run([f"{LLVM}/clang-offload-bundler", "--type=o", "--targets=hipv4-amdgcn-amd-amdhsa--gfx950",
                    f"--input={fat}", f"--output={co}", "--unbundle"], check=True, capture_output=True)
    res = subprocess.run([f"{LLVM}/llvm-objdump", "-d", "--mcpu=gfx950", co], check=True, capture_output=True,
                         text=True)
    return res.stdout


def parse(text):
    """{function: [(addr, mnemonic, args, target_addr or None)]}"""
    funcs, cur, base = {}, None, {}
    for line in text.splitlines():
        m = FUNC.match(line)
        if m:
            cur = m.group(2)
            base[cur] = int(m.group(1), 16)
            funcs[cur] = []
            continue
        m = INSN.match(line)
        if m and cur:
            mnem, args, addr, tail = m.group(1), m.group(2), int(m.group(3), 16), m.group(4)
            tgt = None
            if mnem.startswith("s_branch") or mnem.startswith("s_cbranch"):
                t = TARGET.search(tail)
                if t and t.group(1) in base:
                    tgt = base[t.group(1)] + int(t.group(2) or "0", 16)
            funcs[cur].append((addr, mnem, args, tgt))
    return funcs


def wait_states(mnem, args):
    if mnem == "s_nop":
        return int(args.split()[0], 0) + 1
    return 1


def check_function(insns):
    idx = {a: i for i, (a, _, _, _) in enumerate(insns)}
    preds = {i: [] for i in range(len(insns))}
    succs = {i: [] for i in range(len(insns))}
    for i, (_, mnem, _, tgt) in enumerate(insns):
        falls = not (mnem == "s_branch" or mnem.startswith("s_endpgm") or mnem.startswith("s_setpc"))
        if falls and i + 1 < len(insns):
            preds[i + 1].append(i)
            succs[i].append(i + 1)
        if tgt is not None and tgt in idx:
            preds[idx[tgt]].append(i)
            succs[i].append(idx[tgt])
    bad = []
    for i, (_, mnem, args, _) in enumerate(insns):
        if not mnem.startswith("v_mfma"):
            continue
        ops = operands(args)
        dst = regs(ops[0])
        src = set()
        for o in ops[1:]:
            src |= regs(o)
        # (1) VALU writes of the sources within PRE_WS wait states before
        stack = [(p, 0) for p in preds[i]]
        seen = set()
        while stack:
            j, ws = stack.pop()
            if ws >= PRE_WS or (j, ws) in seen:
                continue
            seen.add((j, ws))
            m2, a2 = insns[j][1], insns[j][2]
            if m2.startswith("v_") and not m2.startswith("v_mfma"):
                o2 = operands(a2)
                # (a swap writes both of its operands)
                written = regs(a2) if "swap" in m2 else (regs(o2[0]) if o2 else set())
                if written & src:
                    bad.append(f"VALU write {m2} {a2} {PRE_WS - ws} wait states before {mnem} {args}")
            stack += [(p, ws + wait_states(m2, a2)) for p in preds[j]]
        # (2) any access to the results within POST_WS wait states after
        stack = [(s, 0) for s in succs[i]]
        seen = set()
        while stack:
            j, ws = stack.pop()
            if ws >= POST_WS or (j, ws) in seen:
                continue
            seen.add((j, ws))
            m2, a2 = insns[j][1], insns[j][2]
            touched = regs(a2)
            if m2.startswith("v_mfma"):
                o2 = operands(a2)
                same_chain = m2 == mnem and o2 and regs(o2[0]) == dst and len(o2) > 3 and regs(o2[3]) == dst
                if (touched & dst) and not same_chain:
                    bad.append(f"{m2} {a2} touches the result of {mnem} {args} after {ws} wait states")
            elif touched & dst and (m2.startswith("v_") or m2.startswith("ds_") or m2.startswith("global_")
                                     or m2.startswith("buffer_") or m2.startswith("scratch_")):
                bad.append(f"{m2} {a2} touches the result of {mnem} {args} after {ws} wait states")
            stack += [(s, ws + wait_states(m2, a2)) for s in succs[j]]
    return bad


def test_hand_written_mfma_hazards(tmp_path):
    if not os.path.exists(OBJ):
        pytest.skip("decode_h128.o not built (run __graft_entry__.build())")
    if not all(os.path.exists(f"{LLVM}/{t}") for t in ("llvm-objcopy", "clang-offload-bundler", "llvm-objdump")):
        pytest.skip("ROCm LLVM tools not found")
    funcs = parse(disassemble(OBJ, str(tmp_path)))
    kernels = {k: v for k, v in funcs.items() if "decode_h128_kernel" in k}
    assert len(kernels) == 4, sorted(funcs)
    report = []
    for name, insns in kernels.items():
        n_mfma = sum(1 for _, m, _, _ in insns if m.startswith("v_mfma"))
        assert n_mfma >= 50, (name, n_mfma)
        report += [f"{name}: {b}" for b in check_function(insns)]
    assert not report, "\n".join(report[:20])


def test_checker_flags_planted_hazards():
    """The checker itself: a VALU write one wait state before an MFMA source
    read, and a VALU read of an MFMA result 5 wait states after it, are caught;
    the same code with enough s_nop passes."""
    def prog(lines):
        return [(4 * i, m, a, None) for i, (m, a) in enumerate(lines)]
    mf = ("v_mfma_f32_32x32x64_f8f6f4", "v[0:15], v[16:23], v[24:31], v[0:15]")
    assert check_function(prog([("v_mov_b32_e32", "v20, v40"), mf, ("s_nop", "15"), ("s_nop", "4")]))
    assert not check_function(prog([("v_mov_b32_e32", "v20, v40"), ("s_nop", "1"), mf, ("s_nop", "15"),
                                    ("s_nop", "4")]))
    assert check_function(prog([("s_nop", "1"), mf, ("s_nop", "3"), ("v_add_f32_e32", "v40, v3, v41")]))
    assert not check_function(prog([("s_nop", "1"), mf, ("s_nop", "15"), ("s_nop", "3"),
                                    ("v_add_f32_e32", "v40, v3, v41")]))
    # an accumulate chain on the same registers needs no wait states
    assert not check_function(prog([("s_nop", "1"), mf, mf, ("s_nop", "15"), ("s_nop", "4")]))
    # a branch back to the MFMA brings the loop's tail into its window
    loop = [("s_nop", "1"), mf, ("s_nop", "15"), ("s_nop", "4"), ("v_mov_b32_e32", "v17, v40"),
            ("s_cbranch_scc1", "")]
    p = prog(loop)
    p[-1] = (p[-1][0], "s_cbranch_scc1", "", 4)
    assert check_function(p)


def _objects(tmp_path):
    if not os.path.isdir(BUILD) or not any(f.endswith(".o") for f in os.listdir(BUILD)):
        pytest.skip("library not built (run __graft_entry__.build())")
    if not all(os.path.exists(f"{LLVM}/{t}") for t in ("llvm-objcopy", "clang-offload-bundler", "llvm-objdump")):
        pytest.skip("ROCm LLVM tools not found")
    out = {}
    for f in sorted(os.listdir(BUILD)):
        if f.endswith(".o"):
            d = tmp_path / f[:-2]
            d.mkdir()
            try:
                out[f] = parse(disassemble(os.path.join(BUILD, f), str(d)))
            except subprocess.CalledProcessError as e:
                if b".hip_fatbin' not found" in (e.stderr or b""):
                    continue  # host code only
                raise
    assert "decode_h128.o" in out and "decode.o" in out, sorted(out)
    return out


def m0_wait_violations(insns):
    """LDS-DMAs issued with no instruction between them and the last M0 write."""
    bad = []
    for i, (_, mnem, args, _) in enumerate(insns):
        if mnem.startswith("global_load_lds") and i > 0:
            pm, pa = insns[i - 1][1], insns[i - 1][2]
            if pm.startswith("s_") and pa.split(",")[0].strip() == "m0":
                bad.append(f"{pm} {pa} directly before {mnem} {args}")
    return bad


FORBIDDEN_SCALAR = ("s_store", "s_buffer_store", "s_scratch_store", "s_atomic", "s_buffer_atomic", "s_dcache_wb")
FORBIDDEN_PACKED = ("v_pk_add_f32", "v_pk_mul_f32", "v_pk_fma_f32")


def test_code_object_rules(tmp_path):
    report = []
    for obj, funcs in _objects(tmp_path).items():
        for name, insns in funcs.items():
            report += [f"{obj} {name}: {b}" for b in m0_wait_violations(insns)]
            for _, mnem, args, _ in insns:
                if mnem.startswith(FORBIDDEN_SCALAR) or mnem in FORBIDDEN_PACKED:
                    report.append(f"{obj} {name}: {mnem} {args}")
    assert not report, "\n".join(report[:20])


def test_m0_rule_checker():
    ok = [(0, "s_mov_b32", "s4, m0", None), (4, "s_mov_b32", "m0, s6", None), (8, "s_mov_b32", "s4, s4", None),
          (12, "global_load_lds_dwordx4", "v[2:3], off", None)]
    bad = [ok[0], ok[1], (8, "global_load_lds_dwordx4", "v[2:3], off", None)]
    assert not m0_wait_violations(ok)
    assert m0_wait_violations(bad)


def kernel_metadata(obj, tmp):
    """[{name, vgpr, agpr, sgpr, scratch, vgpr_spill, sgpr_spill, lds}] from
    the AMDGPU metadata note of the gfx950 code object in a built .o (None
    for a host-only object)."""
    fat = os.path.join(tmp, "fat.bin")
    co = os.path.join(tmp, "dev.co")
    r = subprocess.run([f"{LLVM}/llvm-objcopy", f"--dump-section=.hip_fatbin={fat}", obj, os.path.join(tmp, "host.o")],
                       capture_output=True)
    if r.returncode != 0:
        if b".hip_fatbin' not found" in r.stderr:
            return None
        raise subprocess.CalledProcessError(r.returncode, r.args, r.stdout, r.stderr)
    subprocess.run([f"{LLVM}/clang-offload-bundler", "--type=o", "--targets=hipv4-amdgcn-amd-amdhsa--gfx950",
                    f"--input={fat}", f"--output={co}", "--unbundle"], check=True, capture_output=True)
    txt = subprocess.run([f"{LLVM}/llvm-readobj", "--notes", co], check=True, capture_output=True, text=True).stdout
    doc = txt.split("AMDGPU Metadata: ", 1)[1]
    doc = doc[:doc.index("\n...")] if "\n..." in doc else doc
    out = []
    for k in yaml.safe_load(doc)["amdhsa.kernels"]:
        out.append(dict(name=k[".name"], vgpr=k[".vgpr_count"], agpr=k.get(".agpr_count", 0), sgpr=k[".sgpr_count"],
                        scratch=k[".private_segment_fixed_size"], vgpr_spill=k[".vgpr_spill_count"],
                        sgpr_spill=k[".sgpr_spill_count"], lds=k[".group_segment_fixed_size"]))
    return out


SCRATCH_CHECKED = ("decode.o", "decode_h128.o", "quant.o", "noalloc.o")
A16W8 = re.compile(r"decode_h16_kernelILi0ELi0ELb[01]ELi2E")


def test_no_scratch_in_the_operator_kernels(tmp_path):
    if not os.path.isdir(BUILD) or not os.path.exists(os.path.join(BUILD, "decode.o")):
        pytest.skip("library not built (run __graft_entry__.build())")
    if not os.path.exists(f"{LLVM}/llvm-readobj"):
        pytest.skip("ROCm LLVM tools not found")
    bad, seen = [], 0
    for obj in SCRATCH_CHECKED:
        path = os.path.join(BUILD, obj)
        if not os.path.exists(path):
            continue
        d = tmp_path / obj[:-2]
        d.mkdir()
        for k in kernel_metadata(path, str(d)) or []:
            seen += 1
            if A16W8.search(k["name"]):
                continue
            if k["scratch"] or k["vgpr_spill"]:
                bad.append(f"{obj} {k['name']}: {k['scratch']} B scratch, {k['vgpr_spill']} VGPRs spilled")
    assert seen >= 20, seen
    assert not bad, "\n".join(bad)


def resources_markdown():
    import shutil

    rows = []
    for obj in sorted(f for f in os.listdir(BUILD) if f.endswith(".o")):
        with tempfile.TemporaryDirectory() as d:
            for k in kernel_metadata(os.path.join(BUILD, obj), d) or []:
                name = k["name"]
                if shutil.which("c++filt"):
                    name = subprocess.run(["c++filt", name], capture_output=True, text=True).stdout.strip()
                rows.append((obj, name, k))
    lines = ["| object | kernel | VGPR | AGPR | SGPR | scratch B/lane | VGPR spills | SGPR spills | LDS B |",
             "|---|---|---|---|---|---|---|---|---|"]
    for obj, name, k in rows:
        lines.append(f"| {obj} | `{name}` | {k['vgpr']} | {k['agpr']} | {k['sgpr']} | {k['scratch']} | "
                     f"{k['vgpr_spill']} | {k['sgpr_spill']} | {k['lds']} |")
    return "\n".join(lines)


if __name__ == "__main__":
    if sys.argv[1:] == ["--resources"]:
        print(resources_markdown())
    else:
        sys.exit("usage: python tests/test_isa_rules.py --resources")

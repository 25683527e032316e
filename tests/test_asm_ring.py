"""Register-ring check of the small-batch GEMM (technograd_amd/csrc/kern_qgemm.hip,
qgemv_k), on the gfx950 assembly hipcc writes for it (no GPU needed).

qgemv_k (and gemv16_k) load their operands with inline-assembly loads the compiler does not
track: it believes a load's destination registers hold their value as soon as
the instruction is issued. A ring register whose load is still in flight must
therefore not be given to any other value, or the load overwrites that value
when it lands. This test walks each qgemv_k instantiation from the last full
wait before its final ring load to the first full wait after it, retiring
loads in order at each vmcnt(N), and fails if an instruction after the final
ring load writes a register that an outstanding load will write. (The kernel
prevents this by reading every ring register after its final wait; without
that, the epilogue's row index was computed into such registers, and the
index was overwritten before the row-info loads used it.) Writes by vector
instructions, LDS reads and other loads all count.

The large-batch kernel (qgemm_k) sets m0 in inline assembly before each of
its global-to-LDS copies; a second test checks that nothing else in that
kernel uses m0."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


def _vregs(tok):
    m = re.match(r"v\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", tok)
    return {int(m.group(1))} if m else set()


def ring_hazards(asm_lines):
    """{kernel: [instructions writing an in-flight ring register]} for every
    qgemv_k, gemv16_k and gemv1_k (all load their operands this way). Ring
    loads are the inline-assembly ones (the compiler marks such text with
    ;;#ASMSTART / ;;#ASMEND); loads the compiler wrote itself are waited for
    by the compiler."""
    found = {}
    starts = [i for i, l in enumerate(asm_lines) if re.match(r"^_Z\S*(qgemv_k|gemv16_k|gemv1_k)\S*:", l)]
    for s in starts:
        e = next(i for i in range(s, len(asm_lines)) if "s_endpgm" in asm_lines[i])
        body, inasm, asm_idx = [], False, set()  # loads written as inline assembly (between the ASMSTART/ASMEND markers)
        for l in asm_lines[s:e]:
            t = l.strip()
            if t.startswith(";;#ASMSTART"):
                inasm = True
            elif t.startswith(";;#ASMEND"):
                inasm = False
            elif t and not t.startswith(";"):
                if inasm:
                    asm_idx.add(len(body))
                body.append(t)
        ring = [i for i, t in enumerate(body) if i in asm_idx and re.match(r"global_load_dwordx[24] v\S+, v\d+, s\[", t)]
        assert ring, "no ring loads found in " + asm_lines[s]
        last = ring[-1]
        w0 = max([i for i in range(last) if "vmcnt(0)" in body[i]] + [0])
        end = next(i for i in range(last, len(body)) if "vmcnt(0)" in body[i])
        out, hits = [], []
        for k in range(w0 + 1, end):
            t = body[k]
            p = re.split(r"[\s,]+", t)
            if p[0] == "s_waitcnt":
                m = re.search(r"vmcnt\((\d+)\)", t)
                if m:
                    n = int(m.group(1))
                    out = out[len(out) - n:] if n < len(out) else out
                continue
            if k > last and len(p) > 1 and any(o for o in out) and (
                    (p[0].startswith("v_") and not p[0].startswith("v_cmp")) or p[0].startswith("ds_read")
                    or p[0].startswith("ds_bpermute") or p[0].startswith("global_load") or p[0].startswith("buffer_load")):
                if any(_vregs(p[1]) & o for o in out):
                    hits.append(t)
            if p[0].startswith("global_load") or p[0].startswith("buffer_load"):
                out.append(_vregs(p[1]))
        found[asm_lines[s].split(":")[0]] = hits
    return found


# instructions that read m0 without naming it (moves indexed by m0, messages,
# LDS-destination loads other than the kernel's copies, interpolation, GWS)
M0_IMPLICIT = re.compile(r"^(v_movrel|s_movrel|s_sendmsg|ds_gws|v_interp|buffer_load\S*.*\blds\b)")


def m0_hazards(asm_lines):
    """{kernel: [instructions that use m0 outside the copy pairs]} for every qgemm_k.

    qgemm_k's copies (copy_to_lds) set m0 in inline assembly right before each
    global_load_lds_dwordx4. The compiler does not know that m0 changes there
    (m0 is a reserved register and cannot be declared clobbered), so any other
    use of m0 by compiled code in the kernel could see a copy's LDS address."""
    found = {}
    starts = [i for i, l in enumerate(asm_lines) if re.match(r"^_Z\S*qgemm_k\S*:", l)]
    for s in starts:
        e = next(i for i in range(s, len(asm_lines)) if "s_endpgm" in asm_lines[i])
        body = [l.strip() for l in asm_lines[s:e] if l.strip() and not l.strip().startswith(";")
                and not l.strip().startswith(".")]
        hits, copies = [], 0
        for k, t in enumerate(body):
            op = t.split()[0]
            if op == "global_load_lds_dwordx4":
                if not (k > 0 and re.match(r"s_mov_b32 m0, s\d+$", body[k - 1])):
                    hits.append(t)
                copies += 1
                continue
            if re.match(r"s_mov_b32 m0, s\d+$", t) and k + 1 < len(body) and body[k + 1].startswith("global_load_lds_dwordx4"):
                continue
            if re.search(r"\bm0\b", t) or M0_IMPLICIT.match(t):
                hits.append(t)
        assert copies, "no LDS copies found in " + asm_lines[s]
        found[asm_lines[s].split(":")[0]] = hits
    return found


@pytest.fixture(scope="module")
def qgemm_asm(tmp_path_factory):
    if not os.path.exists(HIPCC) and not shutil.which("hipcc"):
        pytest.skip("hipcc not installed")
    csrc = os.path.join(ROOT, "technograd_amd", "csrc")
    asm = tmp_path_factory.mktemp("asm") / "kern_qgemm.s"
    subprocess.run([HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-ffp-contract=off", "-fno-gpu-flush-denormals-to-zero",
                    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-I", os.path.join(ROOT, "include"), "-I", csrc,
                    "--cuda-device-only", "-S", os.path.join(csrc, "kern_qgemm.hip"), "-o", str(asm)], check=True, capture_output=True)
    return asm.read_text().split("\n")


def test_qgemv_ring_registers_not_reused_in_flight(qgemm_asm):
    found = ring_hazards(qgemm_asm)
    assert sum("qgemv_k" in k for k in found) >= 6 and sum("gemv16_k" in k for k in found) >= 11 and sum(
        "gemv1_k" in k for k in found) >= 10  # every instantiation the launchers use
    bad = {k: v for k, v in found.items() if v}
    assert not bad, bad


def spills(asm_lines, pattern):
    """{kernel: (sgpr spills, vgpr spills)} from the code object metadata of kernels matching pattern."""
    out, name = {}, None
    for l in asm_lines:
        m = re.match(r"\s*(?:- )?\.name:\s+(\S+)", l)
        if m:
            name = m.group(1) if re.search(pattern, m.group(1)) else None
            continue
        m = re.match(r"\s*\.(sgpr|vgpr)_spill_count:\s+(\d+)", l)
        if m and name:
            s, v = out.get(name, (0, 0))
            out[name] = (s + int(m.group(2)), v) if m.group(1) == "sgpr" else (s, v + int(m.group(2)))
    return out


def lane_spills_before_ring_end(asm_lines, name):
    """SGPR spill moves (v_writelane / v_readlane) of kernel `name` that come
    before the first full wait after its last inline-assembly ring load."""
    s = next(i for i, l in enumerate(asm_lines) if l.startswith(name + ":"))
    e = next(i for i in range(s, len(asm_lines)) if "s_endpgm" in asm_lines[i])
    body = [l.strip() for l in asm_lines[s:e] if l.strip() and not l.strip().startswith(";")]
    last = max(i for i, t in enumerate(body) if re.match(r"global_load_dwordx[24] v\S+, v\d+, s\[", t))
    end = next(i for i in range(last, len(body)) if "vmcnt(0)" in body[i])
    return [t for t in body[:end] if t.startswith("v_writelane") or t.startswith("v_readlane")]


def test_inline_load_kernels_do_not_spill(qgemm_asm):
    """A register spilled while its inline-assembly load is in flight is
    stored before the load lands (the compiler believes it already holds the
    value): no instantiation of the kernels that load this way may spill a
    vector register. (An int8 gemv16_k at sixteen waves of eight steps did,
    and computed wrong sums; it is no longer instantiated.) Scalar registers
    spill into lanes of a vector register the compiler sets aside, not to
    memory, and no inline-assembly load targets scalar registers; such
    spills are allowed only after the kernel's last ring load has landed
    (the single-row kernel's resolve of a candidate row, after its product),
    and the ring test above catches a lane write to an in-flight register."""
    found = spills(qgemm_asm, r"(qgemv_k|gemv16_k|gemv1_k)")
    assert len(found) >= 41
    bad = {k: v for k, v in found.items() if v[1] != 0}
    assert not bad, bad
    early = {k: lane_spills_before_ring_end(qgemm_asm, k) for k, v in found.items() if v[0]}
    assert not any(early.values()), early
    assert all("gemv1_k" in k and "Lb1E" in k for k in early), list(early)  # only the fused single-row kernel


def test_inline_loads_take_a_scalar_base(qgemm_asm):
    """The inline-assembly loads name their base address with an "s"
    constraint; when the compiler holds that (uniform) pointer in vector
    registers instead, the listing still prints, but the assembler rejects
    the instruction. Every such load in the listing has a scalar base."""
    bad = [l.strip() for l in qgemm_asm if re.match(r"\s*global_load_dwordx[24] v\[[0-9:]+\], v[0-9]+, v\[", l)]
    assert not bad, bad[:4]


def test_qgemm_m0_only_set_for_lds_copies(qgemm_asm):
    found = m0_hazards(qgemm_asm)
    assert len(found) >= 2  # the int4 and int8 instantiations
    bad = {k: v for k, v in found.items() if v}
    assert not bad, bad


def test_m0_check_sees_a_foreign_use():
    """The m0 scan flags an m0 read that is not one of the copy pairs."""
    lines = ["_Z7qgemm_kILi4EEvv:", "s_mov_b32 m0, s4", "global_load_lds_dwordx4 v1, s[2:3]",
             "s_mov_b32 m0, s5", "v_readlane_b32 s6, v2, m0", "s_endpgm"]
    assert m0_hazards(lines) == {"_Z7qgemm_kILi4EEvv": ["s_mov_b32 m0, s5", "v_readlane_b32 s6, v2, m0"]}

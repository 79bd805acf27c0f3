"""CPU checks over the HIP sources of the library.

Vector-memory instructions issued from inline asm (the direct global->LDS loads
of the K/V loader) are invisible to the compiler's hazard recognizer, so it
inserts no wait states for their scalar operands.  When the SGPR base of such
a load has just been written by a VALU instruction (a v_readlane reload of a
spilled SGPR), gfx950 needs 5 wait states before the load reads it; without
them the load may read a stale base, i.e. a wild address.  Every such asm
statement must therefore put an ``s_nop 4`` (or longer) directly before the
memory instruction.  This test keeps that guard from being dropped.
"""
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "ascend-rsfa_amd", "csrc")

VMEM = re.compile(r"^(global|buffer|flat|scratch)_(load|store|atomic)\w*")
NOP = re.compile(r"^s_nop\s+(\d+)")
ASM = re.compile(r"\basm\s*(?:volatile|__volatile__)?\s*\(((?:\s*\"(?:[^\"\\]|\\.)*\")+)")
STRING = re.compile(r"\"((?:[^\"\\]|\\.)*)\"")


def asm_templates(text):
    """The template string of every asm statement in C++ source text."""
    for m in ASM.finditer(text):
        yield "".join(STRING.findall(m.group(1)))


def unguarded(template):
    """Vector-memory instructions of one asm template not directly preceded by
    s_nop 4 or longer."""
    insts = [i.strip() for i in re.split(r"\\n|\\t|;|\n", template) if i.strip()]
    bad = []
    for n, inst in enumerate(insts):
        if VMEM.match(inst):
            prev = NOP.match(insts[n - 1]) if n > 0 else None
            if prev is None or int(prev.group(1)) < 4:
                bad.append(inst)
    return bad


def test_checker_flags_a_missing_guard():
    src = ('asm volatile("s_nop 0\\n\\tglobal_load_lds_dwordx4 %0, %1" : : "v"(a), "s"(b));\n'
           'asm volatile("buffer_load_dword %0, %1" : "=v"(x) : "v"(y));\n'
           'asm volatile("s_nop 4\\n\\tglobal_load_lds_dwordx4 %0, %1" : : "v"(a), "s"(b));\n')
    found = [unguarded(t) for t in asm_templates(src)]
    assert [len(f) for f in found] == [1, 1, 0]


def test_every_inline_asm_vector_memory_instruction_is_guarded():
    checked = 0
    for name in sorted(os.listdir(CSRC)):
        if not name.endswith((".hip", ".hpp", ".h", ".cpp")):
            continue
        text = open(os.path.join(CSRC, name)).read()
        for t in asm_templates(text):
            assert not unguarded(t), f"{name}: inline asm {t!r} lacks s_nop 4 before its memory instruction"
            checked += sum(1 for i in re.split(r"\\n|\\t|;", t) if VMEM.match(i.strip()))
    # the K/V loader's direct loads are issued from inline asm: the scan must see them
    assert checked >= 1

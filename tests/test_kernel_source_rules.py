"""Rules the HIP kernel sources keep, checked on the text (CPU only).

No VALU instruction is written as inline asm.  An MFMA that reads a VGPR a
VALU instruction wrote needs two wait states between them; the compiler
inserts them after the instructions it emits, but it does not know what an
inline-asm block writes, so an MFMA can follow it too early and read the old
value.  (This happened: the nibble unpack's v_and_or_b32, written as inline
asm, sat one instruction before the MFMA that read it in the W4A16 kernels.)
Inline asm is kept for what has no builtin: waits, the SGPR constant, LDS
DMA with its own M0 set-up, and the LDS-read floor whose loads complete
(s_waitcnt) inside the block."""
import glob
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SOURCES = sorted(glob.glob(os.path.join(ROOT, "rust-gpu_amd", "csrc", "kernels", "*.hip")) +
                 glob.glob(os.path.join(ROOT, "rust-gpu_amd", "csrc", "kernels", "*.h")))


def asm_blocks(text):
    """The instruction text of every asm(...) / asm volatile(...) statement."""
    out = []
    for m in re.finditer(r"\basm\s*(?:volatile\s*)?\(", text):
        depth, i = 1, m.end()
        while depth and i < len(text):
            depth += {"(": 1, ")": -1}.get(text[i], 0)
            i += 1
        body = text[m.end():i - 1]
        code = body.split(":")[0]
        out.append("".join(re.findall(r'"((?:[^"\\]|\\.)*)"', code)))
    return out


def valu_in(asm_text):
    return [t for t in re.findall(r"\b(v_\w+)", asm_text)]


def test_no_valu_instruction_in_inline_asm():
    bad = []
    for path in SOURCES:
        for block in asm_blocks(open(path).read()):
            if valu_in(block):
                bad.append((os.path.basename(path), block))
    assert not bad, bad


def test_the_rule_sees_a_valu_in_inline_asm():
    snippet = 'uint32_t r; asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "s"(m), "v"(b));'
    assert valu_in(asm_blocks(snippet)[0]) == ["v_and_or_b32"]
    assert asm_blocks('asm volatile("s_waitcnt vmcnt(%0)" :: "n"(N) : "memory");') == ["s_waitcnt vmcnt(%0)"]

"""Source checks over the HIP kernels (no GPU).

Vector elements are read through a scalar before a bit cast: this clang
lowers __builtin_bit_cast(T, v[e]) on an element of a clang vector (the
vector_size / ext_vector_type typedefs of csrc) to a read of element 0, and a
queue entry read that way once built a store address from the wrong lane and
faulted the GPU. The check finds every bit cast whose operand subscripts a
name declared with a vector type deeper than that name's array rank."""
import glob
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "alveare_amd", "csrc")


def _sources():
    return {p: open(p).read() for p in sorted(glob.glob(os.path.join(CSRC, "*.hip")) + glob.glob(os.path.join(CSRC, "*.h")))}


def _vector_types(srcs):
    names = set()
    for text in srcs.values():
        names.update(re.findall(r"typedef\s+[\w\s]+?\s+(\w+)\s+__attribute__\(\((?:__vector_size__|ext_vector_type)", text))
    return names


def _vector_names(text, vtypes):
    """name -> array rank of every declaration with a vector element type."""
    ranks = {}
    vt = "|".join(sorted(vtypes))
    for m in re.finditer(r"\b(?:%s)\s*(?:&\s*)?(\w+)((?:\[[^\]]*\])*)" % vt, text):
        ranks[m.group(1)] = max(ranks.get(m.group(1), 0), m.group(2).count("["))
    for m in re.finditer(r"\b(?:%s)\s*\(\s*&\s*(\w+)\s*\)((?:\[[^\]]*\])+)" % vt, text):
        ranks[m.group(1)] = max(ranks.get(m.group(1), 0), m.group(2).count("["))
    return ranks


def violations(srcs):
    vtypes = _vector_types(srcs)
    assert {"u32x4", "f32x4", "bf16x8"} <= vtypes, vtypes
    bad = []
    for path, text in srcs.items():
        ranks = _vector_names(text, vtypes)
        for m in re.finditer(r"__builtin_bit_cast\(\s*[^,()]+(?:\([^()]*\))?\s*,\s*(\w+)((?:\[[^\]]*\])+)\s*\)", text):
            name, subs = m.group(1), m.group(2).count("[")
            if name in ranks and subs > ranks[name]:
                line = text.count("\n", 0, m.start()) + 1
                bad.append(f"{os.path.basename(path)}:{line}: {m.group(0)}")
    return bad


def test_no_bit_cast_of_vector_elements():
    bad = violations(_sources())
    assert not bad, "bit casts of vector elements (read the element through a scalar first):\n" + "\n".join(bad)


def test_check_catches_the_pattern():
    """A planted occurrence of the faulting form is found; the scalar form and
    bit casts of whole vectors are not."""
    src = {
        os.path.join(CSRC, "q4_device.h"): open(os.path.join(CSRC, "q4_device.h")).read(),
        "planted.hip": (
            "__device__ void f(const u32x4 (&q)[5], u32x4 v, float* o) {\n"
            "    o[0] = __builtin_bit_cast(float, v[2]);\n"          # element of a vector: flagged
            "    o[1] = __builtin_bit_cast(float, q[1][3]);\n"       # element of an array's vector: flagged
            "    o[2] = __builtin_bit_cast(float, (uint32_t)v[2]);\n"  # through a scalar: fine
            "    f32x4 w = __builtin_bit_cast(f32x4, q[1]);\n"       # a whole vector: fine
            "}\n"),
    }
    bad = violations(src)
    assert len(bad) == 2 and all("planted.hip" in b for b in bad), bad

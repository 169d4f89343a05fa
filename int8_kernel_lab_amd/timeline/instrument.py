"""Clock-stamped copies of kernel_rowpass.hip and kernel_deepk.hip, and the
build of libi8conv_timeline.so from them (see the package docstring).

Stamps go to a device buffer of [workgroup][16 waves][32 slots] uint64
(s_memrealtime ticks, 100 MHz), written by lane 0 of each wave with plain
vector stores; a null buffer (the default) writes nothing.  Each edit below
must match the current source exactly once, so an edit that no longer
applies fails loudly instead of timing a different kernel.
"""
from __future__ import annotations

import os
import shutil
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
CSRC = os.path.join(PKG, "csrc")
INCLUDE = os.path.join(os.path.dirname(PKG), "include")
BUILD = os.path.join(HERE, "_build")
LIBRARY = os.path.join(BUILD, "libi8conv_timeline.so")

WAVES = 16   # wave slots per workgroup in the stamp buffer
SLOTS = 32   # stamp slots per wave

# Row kernel with copy waves: slot -> meaning
ROWPASS_SLOTS = {0: "wave start", 1: "MFMA wave: arguments loaded", 31: "past the flag barrier",
                 2: "copy wave: all copies issued", 3: "copy wave: copies landed",
                 27: "MFMA wave: walk start", 29: "MFMA wave: walk end",
                 30: "MFMA wave: stores drained"}
ROWPASS_SLOTS.update({4 + r: f"MFMA wave: input row {r} ready" for r in range(10)})
ROWPASS_CYCLES = (26, 28)  # s_memtime at walk start / end (shader clock cycles)
# Deep-channel split-K: slot -> meaning
DEEPK_SLOTS = {0: "wave start", 1: "MFMA wave: arguments loaded", 3: "copy wave: plane loads issued",
               20: "copy wave: planes written", 21: "MFMA wave: halo zeroed",
               23: "MFMA wave: filter landed", 24: "MFMA wave: stores drained"}
DEEPK_SLOTS.update({4 + k: f"copy wave: image {k} flagged" for k in range(16)})
DEEPK_FRAG_SLOTS = {4 + i: f"MFMA wave: fragment {i} image ready" for i in range(8)}

_STAMP = """
__device__ __forceinline__ void tl_put(unsigned long long *tl, int slot, unsigned long long v) {
  if (tl && (threadIdx.x & 63) == 0 && (threadIdx.x >> 6) < %(waves)d)
    tl[(((blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x) * %(waves)d +
        (threadIdx.x >> 6)) * %(slots)d + slot] = v;
}
__device__ __forceinline__ unsigned long long tl_now() { return __builtin_amdgcn_s_memrealtime(); }
""" % {"waves": WAVES, "slots": SLOTS}

ROWPASS_EDITS = [
    ("  int spin_limit;    // polls of a bounded chunk wait (wait_spin_limit())\n};",
     "  int spin_limit;    // polls of a bounded chunk wait (wait_spin_limit())\n"
     "  unsigned long long *tl;\n};"),
    ("constexpr int kStoreElem = 0, kStoreVec = 1, kStoreFull = 2;",
     "constexpr int kStoreElem = 0, kStoreVec = 1, kStoreFull = 2;\n" + _STAMP),
    ("      constexpr int fy_next = IR + 1 - OLO;",
     "      tl_put(p.tl, 4 + G * 10 + IR + 1, tl_now());\n      constexpr int fy_next = IR + 1 - OLO;"),
    ("    flag_wait(counter<G>(p, OLO), p.spin_limit);\n    peeked",
     "    flag_wait(counter<G>(p, OLO), p.spin_limit);\n"
     "    tl_put(p.tl, 4 + G * 10 + OLO, tl_now());\n"
     "    tl_put(p.tl, 26, __builtin_amdgcn_s_memtime());\n"
     "    tl_put(p.tl, 27, tl_now());\n    peeked"),
    ("    st.template store_row<OHI - 1>(p, M != kStoreElem, rows_out, m_row0, oc0, lane);\n  };",
     "    tl_put(p.tl, 28, __builtin_amdgcn_s_memtime());\n"
     "    tl_put(p.tl, 29, tl_now());\n"
     "    st.template store_row<OHI - 1>(p, M != kStoreElem, rows_out, m_row0, oc0, lane);\n"
     "    asm volatile(\"s_waitcnt vmcnt(0)\" ::: \"memory\");\n"
     "    tl_put(p.tl, 30, tl_now());\n  };"),
    ("  const PassArgs &p = p_arg;\n",
     "  const unsigned long long t_start = tl_now();\n  const PassArgs &p = p_arg;\n"),
    ("  // the remaining arguments, in one batch, while the first chunk lands\n  pin_sgprs(p);\n",
     "  // the remaining arguments, in one batch, while the first chunk lands\n  pin_sgprs(p);\n"
     "  tl_put(p.tl, 0, t_start);\n  tl_put(p.tl, 1, tl_now());\n"),
    ("  flag_barrier();\n  run_walk<",
     "  flag_barrier();\n  tl_put(p.tl, 31, tl_now());\n  run_walk<"),
    ("    auto signal = [&](int c) {\n"
     "      if (lane == 0) lds_copy4(one, flags + 16u * uint32_t(c) + 4u * uint32_t(wave), 0u);\n"
     "    };",
     "    auto signal = [&](int c) {\n"
     "      if (lane == 0) lds_copy4(one, flags + 16u * uint32_t(c) + 4u * uint32_t(wave), 0u);\n"
     "      if (c == 0) { tl_put(p.tl, 31, tl_now()); tl_put(p.tl, 0, t_start); }\n"
     "      if (c == nchunks - 1) tl_put(p.tl, 2, tl_now());\n"
     "    };"),
    ("    asm volatile(\"s_waitcnt lgkmcnt(0)\" ::: \"memory\");\n    // the copy wave's work is done",
     "    asm volatile(\"s_waitcnt lgkmcnt(0)\" ::: \"memory\");\n"
     "    tl_put(p.tl, 3, tl_now());\n    // the copy wave's work is done"),
    ("                           : dim3(unsigned(p.tiles_n), unsigned(p.ranges), unsigned(a.n));\n",
     "                           : dim3(unsigned(p.tiles_n), unsigned(p.ranges), unsigned(a.n));\n"
     "  h.tl = size_t(a.n) * size_t(p.ranges) * size_t(p.tiles_n) <= size_t(g_i8_timeline_wgs)\n"
     "             ? g_i8_timeline : nullptr;\n"),
    ("namespace i8conv {\n\n// Set by a wave of rowpass_kernel",
     "namespace i8conv {\nunsigned long long *g_i8_timeline = nullptr;\nint g_i8_timeline_wgs = 0;\n\n"
     "// Set by a wave of rowpass_kernel"),
]
ROWPASS_TAIL = """
// Points the stamps of later launches at buffer, which holds workgroups *
// WAVES * SLOTS uint64; a launch of a larger grid (or a null buffer) stamps
// nothing.
extern "C" void i8conv_timeline_set(void *buffer, int workgroups) {
  i8conv::g_i8_timeline = static_cast<unsigned long long *>(buffer);
  i8conv::g_i8_timeline_wgs = buffer ? workgroups : 0;
}
"""

DEEPK_EDITS = [
    ("  int spin_limit;   // polls of about 64 cycles each per bounded wait (wait_spin_limit())",
     "  int spin_limit;   // polls of about 64 cycles each per bounded wait (wait_spin_limit())\n"
     "  unsigned long long *tl;"),
    ("__device__ __forceinline__ bool flags_set(v4i f) {", _STAMP + "__device__ __forceinline__ bool flags_set(v4i f) {"),
    ("  (void)p_arg;  // read through deep_args() on the MFMA waves' path only\n",
     "  const unsigned long long t_start = tl_now();\n  (void)p_arg;\n"),
    ("  const DeepArgs p = deep_args();\n  pin_sgprs(p);\n",
     "  const DeepArgs p = deep_args();\n  pin_sgprs(p);\n"
     "  tl_put(p.tl, 0, t_start);\n  tl_put(p.tl, 1, tl_now());\n"),
    ("                               : kOutOfRange);\n    }\n    auto signal_ds = [&](int k) {\n",
     "                               : kOutOfRange);\n    }\n    const DeepArgs p = deep_args();\n"
     "    tl_put(p.tl, 0, t_start);\n    tl_put(p.tl, 3, tl_now());\n"
     "    auto signal_ds = [&](int k) {\n"),
    ("    auto signal_ds = [&](int k) {\n      if (lane == 0)\n        asm volatile(\"ds_write_b32",
     "    auto signal_ds = [&](int k) {\n"
     "      tl_put(p.tl, 4 + (k - 1) % 16, tl_now());\n      if (lane == 0)\n        asm volatile(\"ds_write_b32"),
    ("    asm volatile(\"s_waitcnt vmcnt(0) lgkmcnt(0)\" ::: \"memory\");\n    return;",
     "    asm volatile(\"s_waitcnt vmcnt(0) lgkmcnt(0)\" ::: \"memory\");\n"
     "    tl_put(p.tl, 20, tl_now());\n    return;"),
    ("  flag_wait(halo_flags, p.spin_limit);", "  flag_wait(halo_flags, p.spin_limit);\n  tl_put(p.tl, 21, tl_now());"),
    ("  flag_wait(flags, p.spin_limit);\n  v4i A[9][2][2];",
     "  flag_wait(flags, p.spin_limit);\n  tl_put(p.tl, 23, tl_now());\n  v4i A[9][2][2];"),
    ("    flag_wait(flags + 16u * uint32_t(need), p.spin_limit);\n    v4i acc[2][2];",
     "    flag_wait(flags + 16u * uint32_t(need), p.spin_limit);\n"
     "    tl_put(p.tl, 4 + i, tl_now());\n    v4i acc[2][2];"),
    ("    store_frag(f, add_wrap4(acc[0][0], acc[0][1]), add_wrap4(acc[1][0], acc[1][1]));\n  }\n}",
     "    store_frag(f, add_wrap4(acc[0][0], acc[0][1]), add_wrap4(acc[1][0], acc[1][1]));\n  }\n"
     "  asm volatile(\"s_waitcnt vmcnt(0)\" ::: \"memory\");\n  tl_put(p.tl, 24, tl_now());\n}"),
    ("  const int64_t grid = int64_t(p.splits) * p.tiles_n;\n",
     "  const int64_t grid = int64_t(p.splits) * p.tiles_n;\n"
     "  h.tl = grid <= int64_t(g_i8_timeline_wgs) ? g_i8_timeline : nullptr;\n"),
    ("__device__ __attribute__((aligned(4))) unsigned int g_deepk_wait_expired;",
     "__device__ __attribute__((aligned(4))) unsigned int g_deepk_wait_expired;\n"
     "extern unsigned long long *g_i8_timeline;\nextern int g_i8_timeline_wgs;"),
]


def _apply(text: str, edits, name: str) -> str:
    for old, new in edits:
        n = text.count(old)
        if n != 1:
            raise RuntimeError(f"timeline: an edit of {name} matches {n} times (expected once): "
                               f"{old[:60]!r}")
        text = text.replace(old, new)
    return text


def instrumented_sources() -> dict:
    """The two stamped kernel sources, by file name."""
    with open(os.path.join(CSRC, "kernel_rowpass.hip")) as f:
        rowpass = _apply(f.read(), ROWPASS_EDITS, "kernel_rowpass.hip") + ROWPASS_TAIL
    with open(os.path.join(CSRC, "kernel_deepk.hip")) as f:
        deepk = _apply(f.read(), DEEPK_EDITS, "kernel_deepk.hip")
    return {"kernel_rowpass.hip": rowpass, "kernel_deepk.hip": deepk}


def library_objects() -> list:
    """Object names of libi8conv.so, from csrc/Makefile's source lists."""
    names, text = [], open(os.path.join(CSRC, "Makefile")).read().replace("\\\n", " ")
    for line in text.splitlines():
        key, sep, value = line.partition(":=")
        if sep and key.strip() in ("HIP_SRCS", "CPP_SRCS"):
            names += [os.path.splitext(v)[0] + ".o" for v in value.split()]
    if not names:
        raise RuntimeError("timeline: no source lists in csrc/Makefile")
    return names


HIPFLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Wall",
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def object_flags() -> dict:
    """Per-object HIPFLAGS additions of csrc/Makefile ("$(BUILD)/x.o ...:
    HIPFLAGS += ..." lines), by source name: the stamped copies are built
    with the same flags as the library's."""
    extra = {}
    for line in open(os.path.join(CSRC, "Makefile")).read().splitlines():
        targets, sep, rest = line.partition(": HIPFLAGS +=")
        if not sep:
            continue
        for t in targets.split():
            if t.startswith("$(BUILD)/") and t.endswith(".o"):
                name = t[len("$(BUILD)/"):-2] + ".hip"
                extra[name] = extra.get(name, []) + rest.split()
    return extra


def build() -> str:
    """Compiles the stamped kernels and links them with the in-tree objects of
    every other source (csrc/_build, from the library's own build) into
    LIBRARY; returns its path."""
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    objdir = os.path.join(CSRC, "_build")
    src = os.path.join(BUILD, "src")
    os.makedirs(src, exist_ok=True)
    procs, objs = [], []
    for name, text in instrumented_sources().items():
        path = os.path.join(src, name)
        with open(path, "w") as f:
            f.write(text)
        obj = os.path.join(BUILD, name.replace(".hip", ".o"))
        objs.append(obj)
        procs.append(subprocess.Popen([hipcc, *HIPFLAGS, *object_flags().get(name, []),
                                       "-I", INCLUDE, "-I", CSRC, "-c", path, "-o", obj]))
    for proc in procs:
        if proc.wait() != 0:
            raise RuntimeError("timeline: compiling a stamped kernel failed")
    stamped = {os.path.basename(o) for o in objs}
    others = [os.path.join(objdir, o) for o in library_objects() if o not in stamped]
    missing = [o for o in others if not os.path.exists(o)]
    if missing:
        raise RuntimeError(f"timeline: {missing[0]} is missing: build the library first")
    subprocess.run([hipcc, "--offload-arch=gfx950", "-shared", "-o", LIBRARY, *objs, *others],
                   check=True)
    shutil.rmtree(src, ignore_errors=True)
    return LIBRARY

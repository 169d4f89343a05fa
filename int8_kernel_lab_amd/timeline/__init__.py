"""Per-wave timelines of the row kernel with copy waves (kernel_rowpass.hip)
and the deep-channel split-K kernel (kernel_deepk.hip): a measurement tool,
not part of the convolution path.

``instrument.write_sources`` writes copies of the two kernel sources with
device clock stamps (s_memrealtime, 100 MHz) at fixed points of each wave's
run (start, arguments loaded, workgroup barrier, copies issued and landed,
each input row or image ready, each filter tap ready, end of the MFMA walk,
stores drained); ``instrument.build`` compiles them with the in-tree
objects of every other source into ``timeline/_build/libi8conv_timeline.so``
(the same C ABI plus ``i8conv_timeline_set``, which points the stamps at a
device buffer).  ``python -m int8_kernel_lab_amd.timeline run`` loads that
library in a child process (I8CONV_LIBRARY), checks the layer against the
oracle, times it like bench.py's graph region and prints the stamps' per-wave
spread (min / median / max, microseconds from the launch's first wave).
"""

"""navi-tts on MI355X: Python plumbing over the gfx950 C ABI (include/navi_amd.h).

The compute lives in navi-tts_amd/lib/libnavi_amd.so (HIP kernels for gfx950) and
the C++ host classes in navi-tts_amd/csrc/host; this package only loads the
library, moves buffers and writes `.navi` blobs.
"""

// Unity device translation unit: every kernel of the library is compiled
// here, so the shared library carries exactly one gfx950 code object.
#include "gemm.hip"
#include "rows.hip"
#include "attention.hip"
#include "vision.hip"
#include "audio.hip"
#include "mel.hip"
#include "search.hip"
#include "noalloc.hip"
#include "probe.hip"

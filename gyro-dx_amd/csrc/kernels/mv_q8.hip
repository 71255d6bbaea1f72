// Q8_0 rows in the repacked layout of q8_repack (the real model's Q8_0 shared expert). See
// mv_common.h; replaces mv_q8 of shaders/engine/mv.hlsl:53-92. Requires cols a multiple of 64
// (src/gpu_engine.zig:294).
#include "mv_common.h"
GD_PIPELINE_NAMED(mv_q8, 256) { mv_body<MV_Q8>(a); }

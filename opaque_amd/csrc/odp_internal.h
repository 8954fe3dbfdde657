// Host-side helpers shared by the entry-point translation units.
#pragma once

#include "odp_common.h"

#define ODP_ABI_VERSION 3

// fp64 partials of the static scratch behind odp_clip_materialized_noalloc
// (8 MiB per GPU).
#define ODP_NOALLOC_MAX_PARTIALS ((int64_t)1 << 20)

void odp_set_error(const char* fmt, ...);
int odp_check_launch(const char* what);
int odp_check_table(const char* what, const void* problems, const int32_t* work_start,
                    int32_t n_prob, int32_t total_blocks);

static inline hipStream_t odp_hip_stream(odp_stream_t s) { return (hipStream_t)s; }

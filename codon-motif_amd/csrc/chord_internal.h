// Chord decode over a device cursor, shared by the C-ABI entry points that take
// a caller workspace and those that use the library's own scratch.
#pragma once

#include <stddef.h>
#include <stdint.h>

namespace motif {

// The body of motif_chord_decode (same arguments and status codes).
int chord_decode_run(
    const void *q, int64_t q_sb, int64_t q_sh, int64_t q_st,
    const void *k_cache, int64_t k_sb, int64_t k_sh, int64_t k_st,
    const void *v_cache, int64_t v_sb, int64_t v_sh, int64_t v_st,
    int *length_dev, int capacity,
    const float *alpha, const float *beta, const float *mu, const float *ssmax,
    const float *log_n, int64_t ln_sb, int64_t ln_st, const float *log_table, int log_table_len,
    void *out, int64_t o_sb, int64_t o_sh, int64_t o_st,
    int B, int H, int Hkv, int L, int D, float scale, float eps,
    void *workspace, size_t workspace_bytes, int dtype, void *stream);

}  // namespace motif

/*
 * rope_tables.c -- host-side RoPE tables (C11).
 *
 * Replaces model.c:545-556 (init_rope_tables): theta = (float)pos /
 * powf(base, (float)(2i)/(float)head_dim), cos/sin via the host libm.  The
 * device never evaluates trigonometry: it reads these tables, so the rotation
 * it applies is bit-identical to the reference's on the same host.  Built with
 * -std=c11 -ffp-contract=off like the reference.
 */
#include <math.h>
#include <stddef.h>

#include "picolm_hip.h"

void plh_rope_tables_host(float *cos_tab, float *sin_tab, int max_seq_len,
                          int head_dim, float freq_base) {
    int half = head_dim / 2;
    for (int p = 0; p < max_seq_len; p++) {
        float *crow = cos_tab + (size_t)p * (size_t)half;
        float *srow = sin_tab + (size_t)p * (size_t)half;
        for (int i = 0; i < half; i++) {
            float inv_freq_div = powf(freq_base, (float)(2 * i) / (float)head_dim);
            float theta = (float)p / inv_freq_div;
            crow[i] = cosf(theta);
            srow[i] = sinf(theta);
        }
    }
}

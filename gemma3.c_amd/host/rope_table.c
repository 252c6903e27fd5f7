/*
 * rope_table.c - g3attn_rope_precompute: the RoPE cos/sin table on the host.
 *
 * Same fp32 expression and libm calls as gemma3_rope_precompute
 * (gemma3_kernels.c:455-468).  The table's low bits depend on how the
 * reference was compiled: gcc -ffast-math vectorises powf/cosf/sinf, so the
 * reference's fast / threads / blas-threads builds (Makefile:32, 58-73) and
 * its plain release build differ by an ulp in some entries.  This file is
 * compiled with the fast-mode flags (see Makefile: -O3 -ffast-math, AVX2) and
 * reproduces those tables bit for bit; g3attn_create uploads whatever table
 * the caller passes, so an engine always gets its own bits.
 */
#include "g3attn.h"

#include <math.h>
#include <stddef.h>

void g3attn_rope_precompute(float *freqs, int max_pos, int head_dim, float theta) {
    const int half = head_dim / 2;
    for (int p = 0; p < max_pos; p++) {
        for (int i = 0; i < half; i++) {
            float inv = 1.0f / powf(theta, (float)(2 * i) / (float)head_dim);
            float ang = (float)p * inv;
            freqs[((size_t)p * half + i) * 2] = cosf(ang);
            freqs[((size_t)p * half + i) * 2 + 1] = sinf(ang);
        }
    }
}

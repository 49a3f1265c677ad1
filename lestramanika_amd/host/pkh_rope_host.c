/*
 * pkh_rope_host.c -- host-side RoPE tables for callers without a
 * pickle_fast_state_t.
 *
 * The formulas are the reference's (src/pickle_fast.c:1638-1640 for the
 * inverse frequencies, src/pickle_fast.c:1779-1786 for the sin/cos rows):
 * the device kernels consume these fp32 bits unchanged, so a caller that
 * builds its tables here gets the same rotation as the reference's state.
 */
#include <math.h>
#include <stdlib.h>

#include "pkh_attn.h"

void pkh_rope_host_tables(int head_dim, float theta, int p_begin, int p_last,
                          float* inv_freq, float* sin_tab, float* cos_tab) {
    int half = head_dim / 2;
    if (half > 64) half = 64;
    if (half <= 0) return;
    float local[64];
    float* f = inv_freq ? inv_freq : local;
    for (int i = 0; i < half; i++)
        f[i] = 1.0f / powf(theta, (float)(2 * i) / (float)head_dim);
    if (!sin_tab || !cos_tab) return;
    for (int p = p_begin; p <= p_last; p++) {
        float* sp = sin_tab + (size_t)p * half;
        float* cp = cos_tab + (size_t)p * half;
        for (int i = 0; i < half; i++) {
            float angle = f[i] * (float)p;
            sp[i] = sinf(angle);
            cp[i] = cosf(angle);
        }
    }
}

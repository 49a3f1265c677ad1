/* A C99 host of the attention library, built by tests/test_abi.py the way
 * pickle would build against it: include pkh_attn.h, link -lpkh.  It only
 * calls entry points that do no device work (version, host RoPE tables,
 * argument checks), so it runs without a GPU. */
#include "pkh_attn.h"

#include <math.h>
#include <stdio.h>
#include <string.h>

int main(void) {
    const char* version = pkh_version();
    if (!version || !strstr(version, "gfx950")) return 1;

    /* Rows 0..3 of the head_dim-128 tables: half = 64, inv_freq[0] = 1,
     * row 0 is sin 0 / cos 1, and row p's first angle is p radians. */
    float inv[64], sn[4 * 64], cs[4 * 64];
    pkh_rope_host_tables(128, 500000.0f, 0, 3, inv, sn, cs);
    if (inv[0] != 1.0f || sn[0] != 0.0f || cs[0] != 1.0f) return 2;
    if (fabsf(sn[2 * 64] - sinf(2.0f)) > 1e-6f || fabsf(cs[3 * 64] - cosf(3.0f)) > 1e-6f) return 3;

    pkh_kv_t kv;
    memset(&kv, 0, sizeof kv);
    if (pkh_kv_alloc(0, 8, 128, 16, PKH_KV_F32, &kv) != PKH_ERR_ARG) return 4;
    if (pkh_attn_decode(NULL, NULL, 0, 0, 32, NULL, NULL, NULL, NULL) != PKH_ERR_ARG) return 5;
    if (pkh_attn_prefill(NULL, NULL, 0, 0, 1, 32, NULL, NULL, NULL, NULL) != PKH_ERR_ARG) return 6;
    pkh_kv_free(&kv);   /* a zeroed struct: no-op */

    printf("c host ok: %s\n", version);
    return 0;
}

/* Layout of the oracle's model state, shared by oracle.c and port32.c -- TEST
 * INFRASTRUCTURE ONLY (see oracle.h). */
#ifndef ICUA_ORACLE_MODEL_H
#define ICUA_ORACLE_MODEL_H
#include "oracle.h"

typedef struct {
    const float *attn_norm, *q_norm, *k_norm, *mlp_norm;
    const uint8_t *wqkv, *wqkv_sb, *wo, *wo_sb, *wgu, *wgu_sb, *wd, *wd_sb;
} or_layer_w;

struct or_model {
    int fmt, layers, maxctx;
    const uint8_t* img;
    const uint8_t *embed, *embed_sb;
    const float* final_norm;
    or_layer_w L[OR_MAXLAYERS];
    uint16_t* kv; /* [layers][2][NKV][maxctx][HD] */
    float* rope;  /* [maxctx][64][2] */
};

#endif

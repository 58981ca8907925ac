// Launch interface of the persistent decode kernel (persist.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "icua_shared.h"

namespace icua {

// Workgroups of the persistent kernel: one per CU of an MI355X.  The static work split
// (16-row blocks of QKV / O / gate|up / down, 32 attention splits per KV group) is built for
// exactly this many.
constexpr int PERSIST_WGS = 256;

struct LayerPtrs {
    const float *attn_norm, *q_norm, *k_norm, *mlp_norm;
    const uint8_t *wqkv, *wqkv_sb, *wo, *wo_sb, *wgu, *wgu_sb, *wd, *wd_sb;
};

struct PersistArgs {
    // Per-layer tensor pointers, held in the kernel arguments so that the kernel reads them with
    // scalar loads: a vector load of a pointer would make the wave wait for every weight tile it
    // has in flight before the address can be formed.
    LayerPtrs layers[MAX_LAYERS];
    int nlayers;
    int nsteps;               // decode steps to run (stops early at a stop condition)
    int maxctx;               // cache capacity (row stride of the K/V cache)
    const uint8_t* E;         // tied embedding / lm_head codes (tiled) and scales
    const uint8_t* Esb;
    const float* final_norm;
    const float* rope;        // [maxctx][64] (cos, sin)
    uint16_t* kv;             // [layers][2][NKV][maxctx][HD] fp16
    float* x;                 // residual rows [2][H]: the next pass's token embeddings, in and out
    State* st;
    int* out_tokens;
    uint64_t* ll;             // packet area of persistent_sync_bytes(), zeroed before the launch
};

// nr = 1: a.nsteps single-token steps (ending early, with the pair pending in the control
// block, when a commit forces a grammar pair); nr = 2: the pending pair as one two-row pass
// (a.nsteps must be 1), which commits the pair's next token.
hipError_t launch_persistent(int fmt, int nr, const PersistArgs& a, hipStream_t s);
// One-token GEMV y[N] = W x (W tiled, q4 or q8, K = 2048 or 6144) on the lm_head stage's
// streaming schedule; hipErrorInvalidValue for other shapes or more than 160 x 256 row blocks.
hipError_t launch_gemv_stream(int fmt, const uint8_t* w, const uint8_t* sb, const float* x, float* y, int N, int K,
                              hipStream_t s);
// Size of the packet area the workgroups exchange data through (zeroed before every launch), and
// the index (in 32-bit words) of its error flag: non-zero after a launch means a wait timed out.
size_t persistent_sync_bytes();
int persistent_error_slot();
// Bytes of the packet area a launch of nr-row passes uses (cleared before it, with the error flag).
size_t persistent_clear_bytes(int nr);

}  // namespace icua

// Definitions shared by the host engine and the kernels.
#pragma once
#include <stdint.h>

namespace icua {

// Language-backbone dimensions (Sources/Engine/ModelFile.swift:47-59; Shaders.swift:23-37).
constexpr int H = 2048;
constexpr int FF = 6144;
constexpr int NH = 16;
constexpr int NKV = 8;
constexpr int HD = 128;
constexpr int QKV = 4096;
constexpr int GU = 12288;
constexpr int VOCAB = 151936;
constexpr int MAX_LAYERS = 28;
constexpr int IMAGE_PAD_ID = 151655;  // Shaders.swift:38
constexpr float EPS = 1e-6f;          // Shaders.swift:36

// Tokens one pass of the GEMV path carries (decode n = 1, grammar pairs n = 2, verify n <= 8).
constexpr int MAXM = 8;
// Workgroups that produce lm_head argmax partials.
constexpr int LMH_WAVES = 1024;

enum WeightFormat { FMT_F16 = 0, FMT_Q8 = 1, FMT_Q4 = 2 };

// Decode control block (Shaders.swift:41-54).  The first twelve fields keep the reference
// layout; the rest are additions of this engine.
struct State {
    int pos;         // cache slot of the first token of the current pass
    int n;           // tokens in the current pass
    int step;        // generated tokens committed so far
    int done;        // stop flag: every kernel returns at once while it is set
    int maxctx;      // cache capacity
    int maxsteps;    // generation limit
    int eos0;        // primary EOS id
    int eos1;        // secondary EOS id
    int vis_offset;  // pass row where the image-pad run starts (-1 if none)
    int n_vis;       // number of visual rows
    int rope_delta;  // M-RoPE delta
    int npatches;    // ViT patches (unused by the decoder)
    int flags;       // STATE_FLAG_* below
    int logits_rows; // 0: argmax only; 1: last-row logits; n: logits of every row
    int pad[2];
};
static_assert(sizeof(State) == 64, "State layout");

constexpr int STATE_FLAG_GRAMMAR = 1;  // grammar pairs and ')' stop of Shaders.swift:1543-1560

}  // namespace icua

// Internal launchers shared by the C-ABI entry points and the decode
// session. The session passes its own scratch buffers so that nothing inside
// a captured token step allocates.
#pragma once

#include "xp_internal.hpp"

namespace xp {

constexpr int kMvMaxMats = 4;
constexpr int kMaxHeadDim = 512;

// ---- int4 matvec ----
struct MvMatDesc {
    float*      out;
    const void* wq;
    const void* sc;
    uint32_t    cols;
};
// Partial floats a call with these shapes needs for a given split (0 = auto).
size_t mv_partial_floats(uint32_t rows, uint32_t total_cols, uint32_t split, int n_cu);
int launch_mv(const MvMatDesc* mats, uint32_t n, const float* x, int fmt, uint32_t rows,
              uint32_t split, float* partial, size_t partial_cap, uint32_t* tickets,
              size_t tickets_cap, hipStream_t st, const char* who);

// ---- QK-norm + RoPE + KV append ----
struct QkArgs {
    float* q_out;
    float* k_out;
    const float* q_raw;
    const float* k_raw;
    const float* v;
    const float* qw;
    const float* kw;
    uint16_t* kcache;
    uint16_t* vcache;
    uint32_t n_heads, kv_heads, head_dim;
    float eps;
    const uint32_t* pos_dev;   // when non-null, the position is read here
    uint32_t pos;
};
int launch_qk(const QkArgs& a, float theta, hipStream_t st);

// ---- decode attention ----
struct AttnArgs {
    float* out;
    const float* q;
    const uint16_t* kc;
    const uint16_t* vc;
    uint32_t n_heads, kv_heads, head_dim, group;
    uint32_t span, kv_start;
    const uint32_t* pos_dev;   // when non-null: span / kv_start derive from it
    uint32_t window;           // 0 = global (with pos_dev)
    float scale;
    uint32_t nsplit;
    float* part;               // [kv_heads][nsplit][group][2 + head_dim]
    uint32_t* tickets;         // [kv_heads]
};
uint32_t attn_splits(uint32_t max_span);
size_t attn_partial_floats(uint32_t kv_heads, uint32_t n_heads, uint32_t head_dim,
                           uint32_t max_span);
int launch_attention(AttnArgs a, uint32_t max_span, hipStream_t st);

// ---- sampling ----
constexpr int kAmMaxWg = 256;
int launch_argmax(uint32_t* out_idx, float* out_val, const float* logits, uint32_t n,
                  float* pval, uint32_t* pidx, uint32_t* ticket, hipStream_t st);
int launch_topk4(float* cval, uint32_t* cidx, const float* x, uint32_t n, uint32_t nparts,
                 hipStream_t st);

}  // namespace xp

// Arguments of the persistent token loop (loop.hip).
#pragma once

#include "launch.h"

namespace bh {

struct LayerDev {
    Packed q, k, v, o, gate, up, down;
    const float* attn_norm;
    const float* q_norm;
    const float* k_norm;
    const float* attn_sub;
    const float* ffn_norm;
    const float* ffn_sub;
    const float* q_bias;  // projection biases or null
    const float* k_bias;
    const float* v_bias;
    int rope;             // 0: the layer attends without RoPE
    uint16_t* kc;  // [kv_heads][ctx][head_dim] fp16
    uint16_t* vc;
    Packed down_t;  // with push_ffn: the down matrix block-major (launch_unit_transpose)
};

struct LoopArgs {
    const LayerDev* layers;  // device array
    int n_layers;
    Packed embd, out;
    const float* out_norm;
    int embd_dim, heads, kv_heads, head_dim, ff, neox, relu2;
    float eps, scale;
    const float* rope;       // [ctx][rope_dim]
    int rope_dim;
    int ctx;
    // tagged hand-off words: (tag << 32) | float bits
    unsigned long long *ht, *qt, *kt, *vt, *attt, *actt, *pacct, *pmlt;
    unsigned long long* sct;   // the spread attention's scores: [kv head][head][position], packed by length
    // exact attention spread over the grid (stage 1 by position chunks, stage 2 by 32-wide value slices)
    int spread;
    // its launch constants: value slices a head, stage-2 workgroups, stage-1 workgroups a key/value
    // head; sp_all: it takes every position of the session's context
    int sp_slices, sp_n2, sp_per_kv, sp_all, sp_hpk;
    unsigned tag_base;
    float* logits;
    int max_splits;
    unsigned long long* keys;  // [2] pick keys, by step parity
    unsigned* done;            // [4] phase-H workgroups done, by step parity (monotonic in a launch)
    int* pos_out;              // device position after the launch
    int* seq;                  // token sequence by position
    int seq_len;
    int fixed;                 // seq[0, fixed) are caller tokens
    int pos0, n_steps, first_full;  // steps >= first_full compute the output projection and pick
    int* error;                // set when a barrier wait expires
    unsigned long long* trace; // optional: wall clocks of the phases (workgroup 0; every workgroup at one step/layer)
    int trace_step, trace_layer;
    int R_qkv[3], tiles_qkv[3];
    int R_o, tiles_o, R_gu, tiles_gu, R_d, tiles_d, R_h, tiles_h;
    // O and down tiles cover the same rows of h on the same workgroup, which
    // then keeps its rows of h in LDS for the residual adds
    int own_h;
    // the O and down tiles (phases C and F) go to workgroups c_first, c_first + 1, ...: with the
    // spread attention the workgroups of its second stage, which finish phase B last, take none
    int c_first;
    int n_c;  // ... and to n_c workgroups from there (round-robin)
    // the attention output is handed to phase C quantised (Q8_0 O matrix, no sub-norm)
    int att_q8;
    // exact attention one workgroup per query head (else one per key/value head)
    int head_attn;
    // the feed-forward block pushed to its consumers: the workgroup of activation block j
    // (gate/up rows 32 j .. 32 j + 31) quantises that block and writes the down matrix's
    // term of block j for every row, dtt[j][row]; the owners of h's rows add them in block
    // order (phase F).  Tasks go to workgroups d_first, d_first + 1, ... (mod the grid).
    int push_ffn, d_first;
    unsigned long long* dtt;
    // resident attention for contexts up to loop_resident_max() positions: workgroups
    // 0 .. res_n - 1 (task: query head, 64-wide value slice) hold the layer's cached keys and
    // their value slice in LDS, loaded while the other phases run, and take the whole attention;
    // they take no tiles of phases A, C, D and F
    int res_ok, res_n;
    // a_touch: before phase F, each h-row owner with a phase-A tile in the next layer loads that
    // tile's bytes once (into L2), so its phase-A weight loads, and the input poll behind them,
    // do not wait for HBM
    int a_touch;
};

constexpr int kOwnRows = 256;  // rows of h one workgroup can keep

int loop_units_per_thread(uint32_t type, bool head);
// Whether the spread exact attention takes this shape on a grid of `grid` workgroups.
bool loop_spread_fits(int heads, int kv_heads, int head_dim, int rope_dim, int grid);
// Whether it takes every position of a context of `positions` (longer ones take the split attention).
bool loop_spread_covers(int heads, int kv_heads, int head_dim, int grid, int positions);
// Whether the pooled exact attention takes every length of a context of `positions`.
bool loop_pool_covers(int hpk, int positions);
// Positions the resident attention takes (the context of a step, this token's included).
int loop_resident_max();

const void* find_loop_kernel(uint32_t tq, uint32_t tv, uint32_t to, uint32_t tg, uint32_t td, uint32_t th);
hipError_t launch_loop(const void* kernel, const LoopArgs& g, int grid, hipStream_t s, bool cooperative);

}  // namespace bh

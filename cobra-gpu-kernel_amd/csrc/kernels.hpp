// Internal launcher interface between the kernels and the C ABI (capi.hip).
// Every launcher validates its arguments, enqueues on the given stream and
// returns a hipError_t; none allocates, frees or synchronises, so each is
// safe to record into a hipGraph.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cobra {

constexpr int kLnMaxD = 4096;  // widest row the LayerNorm kernels hold in registers

// Row-mask and activation options of the GEMM epilogues (bit flags, applied
// in this order; mask byte 0 = padded row, any other value = valid row).
enum : int {
  kEpiGelu = 1,        // v = gelu(v) with the exact erf form, after the bias
  kEpiMaskBranch = 2,  // padded rows: v = 0 before the residual add (masked_fill of the branch)
  kEpiMaskResid = 4,   // padded rows: (v + resid) * 0 -- the reference epilogue's MASK_RESID
  kEpiMaskOut = 8,     // LayerNorm epilogue: padded rows' normalised output * 0 (MASK_OUT)
};

struct LnArgs {
  const void* x;           // [rows, d], x_dtype (kF16, kF32 or kBF16; y_dtype likewise)
  int x_dtype;
  const void* branch;      // optional [rows, d] added to x before the norm
  int branch_f32;          // branch dtype: 1 = fp32, 0 = fp16
  const float* gamma;      // [d]
  const float* beta;       // [d]
  float* resid_out;        // optional [rows, d] fp32 store of x (+ branch)
  void* y;                 // [rows, d], y_dtype
  int y_dtype;
  int64_t rows;
  int d;
  float eps;
  hipStream_t stream;
  const uint8_t* row_mask = nullptr;  // optional [rows]; 0 = padded row
  int mask_resid = 0;      // r *= mask before the store and the statistics
  int mask_out = 0;        // y *= mask
  // Row strides in elements (0 = d) and zero fill: with ldy > d, y columns d .. ldy-1
  // are written as 0 (a row padded for the GEMM that consumes it).  Any stride or a
  // width that is not a multiple of 8 takes the element-wise kernel.
  int64_t ldx = 0, ldb = 0, ldr = 0, ldy = 0;
};
hipError_t run_ln(const LnArgs& a);

// Weights of the padded staged plan (head_dim or d_model not a multiple of 8):
//   out[r][c] = in[rmap(r)][cmap(c)], 0 where a map has no source;
// a map takes i -> (i / gout) * gin + i % gout when i % gout < gin and that is < lim.
struct PadArgs {
  const void* in;   // [in_rows, in_cols] row-major
  void* out;        // [out_rows, out_cols] row-major
  int elem_bytes;   // 2 (fp16) or 4 (fp32)
  int64_t in_cols, out_rows, out_cols;
  int64_t r_gin, r_gout, r_lim;
  int64_t c_gin, c_gout, c_lim;
  hipStream_t stream;
};
hipError_t run_pad(const PadArgs& a);

struct GemmArgs {
  const void* a;           // [M, K] ab_dtype, row-major
  const void* w;           // [N, K] ab_dtype (nn.Linear layout)
  const float* bias;       // optional [N] fp32
  const void* resid;       // optional [M, N] added in the epilogue
  int resid_dtype;
  void* c;                 // [M, N] c_dtype; with the LN epilogue: optional fp32 residual store
  int c_dtype;
  int64_t M;
  int N;
  int K;
  const float* ln_gamma;   // non-null selects the LayerNorm epilogue (requires N <= 128)
  const float* ln_beta;
  void* ln_y;              // [M, N] LayerNorm output
  int ln_y_dtype;
  float eps;
  hipStream_t stream;
  const uint8_t* row_mask = nullptr;  // [M] when a kEpiMask* flag is set
  int epi = 0;             // kEpi* flags
  // Operand type of a and w: kF16, or kBF16 (then resid, c and ln_y are kBF16 or kF32,
  // and the LayerNorm epilogue is the K, N in {64, 128} kernel's only).
  int ab_dtype = 0;  // kF16
};
// Compute units of the current device (cached after the first call).
inline int compute_units() {
  static int n = 0;
  if (n == 0) {
    int dev = 0, v = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
      n = v;
    else
      n = 256;
  }
  return n;
}

hipError_t run_gemm(const GemmArgs& a);
// Plain-epilogue GEMMs through LDS-DMA tiles (K % 64 == 0, N % 8 == 0, at
// least half a round of 128 x 128 tiles); run_gemm routes eligible shapes there.
bool gemm_dma_ok(const GemmArgs& a);
hipError_t run_gemm_dma(const GemmArgs& a);

// Out-projection with LayerNorm over rows of N = 256 .. 2048 in its epilogue
// (gemm_dma.hip): y = LN(x + mask(a W^T + bias)) * gamma + beta, a / w / x / y all fp16 or
// all bf16.
// The column tiles of a row block exchange per-row statistics through `sync`
// (gemm_rowln_sync_bytes, 64-bit words that must all hold kRowLnUnset at launch), so
// the whole grid has to fit the chip at once: gemm_rowln_ok.  Launches that share a
// sync area must not overlap.
constexpr uint64_t kRowLnUnset = ~0ull;
struct GemmRowLnArgs {
  const void* a;           // [M, K] dtype
  const void* w;           // [N, K] dtype
  const float* bias;       // [N]
  const void* x;           // [M, N] dtype residual
  const float* gamma;      // [N]
  const float* beta;       // [N]
  void* y;                 // [M, N] dtype
  int64_t M;
  int N;
  int K;
  float eps;
  const uint8_t* row_mask; // optional [M]: 0 = padded row, whose branch is zeroed
  void* sync;
  hipStream_t stream;
  int dtype = 0;           // a, w, x and y: kF16 (0) or kBF16
};
bool gemm_rowln_ok(int64_t M, int N, int K);
int64_t gemm_rowln_sync_bytes(int64_t M, int N);
hipError_t run_gemm_rowln(const GemmRowLnArgs& a);

// LayerNorm in the prologue of the projection that consumes it (ln_gemm.hip):
// c = (LayerNorm(x) * gamma + beta) w^T + bias, rows of d = 64 or 128, fp16 out.
struct LnGemmArgs {
  const void* x;           // [M, d], x_dtype
  int x_dtype;
  const float* gamma;      // [d]
  const float* beta;       // [d]
  const void* w;           // [N, d], ab_dtype
  const float* bias;       // optional [N]
  void* c;                 // [M, N], ab_dtype
  int64_t M;
  int N;
  int64_t d;
  float eps;
  hipStream_t stream;
  int ab_dtype = 0;        // operands and output: kF16, or kBF16 (x then bf16 or fp32)
};
bool ln_gemm_ok(int64_t d, int x_dtype, int ab_dtype = 0);
hipError_t run_ln_gemm(const LnGemmArgs& a);
// LayerNorm epilogue for K = 64 / 128 and N = 64 / 128 (ln_gemm.hip); run_gemm
// routes eligible calls there.
bool gemm_ln_rows_ok(const GemmArgs& a);
hipError_t run_gemm_ln_rows(const GemmArgs& a);

struct AttnArgs {
  const void* qkv;         // [B*S, 3*H*hd] dtype: q | k | v column blocks, head-major inside each
  void* ctx;               // [B*S, H*hd] dtype
  int64_t batch;
  int seq_len;
  int heads;
  int head_dim;
  float scale;             // softmax scale (head_dim ** -0.5 in the layer)
  int causal;
  hipStream_t stream;
  const uint64_t* key_bits = nullptr;  // optional [batch][ceil(S/64)]: bit j of word w = key 64w+j valid
  int dtype = 0;           // element type of qkv and ctx: kF16 (0) or kBF16
};
hipError_t run_attn(const AttnArgs& a);

// QKV projection fused into exact attention, one workgroup per (sequence, head):
// head_dim 256, S <= 128 (qkv_attn.hip).  ctx must not overlap h.
struct QkvAttnArgs {
  const void* h;           // [B*S, D] dtype (D = heads * head_dim)
  const void* w_qkv;       // [3D, D] dtype: q | k | v rows
  const float* b_qkv;      // [3D] or null
  void* ctx;               // [B*S, D] dtype
  int64_t batch, seq_len, heads, head_dim;
  float scale;
  int causal;
  const uint64_t* key_bits;  // optional [batch][ceil(S/64)]
  hipStream_t stream;
  uint64_t* fill = nullptr;  // optional: nfill words set to kRowLnUnset (for the kernel that follows)
  int64_t nfill = 0;
  int dtype = 0;             // h, w_qkv and ctx: kF16 (0) or kBF16
};
bool qkv_attn_head_ok(int64_t seq_len, int64_t heads, int64_t head_dim);
hipError_t run_qkv_attn_head(const QkvAttnArgs& a);

// mask [batch, S] bytes (0 = padded) -> key_bits [batch][ceil(S/64)] (attn.hip).
hipError_t run_mask_bits(const uint8_t* mask, uint64_t* bits, int64_t batch, int seq_len, hipStream_t stream);
inline int64_t mask_words(int64_t seq_len) { return (seq_len + 63) / 64; }

// Whole sublayer in one kernel (layer_small.hip).
struct SmallLayerArgs {
  const void* x;           // [B*S, D], x_dtype
  int x_dtype;
  const void* w_qkv;       // [3D, D] fp16
  const float* b_qkv;      // [3D]
  const void* w_o;         // [D, D] fp16
  const float* b_o;        // [D]
  const float* ln1_w;
  const float* ln1_b;
  const float* ln2_w;
  const float* ln2_b;
  void* y;                 // [B*S, D], x_dtype
  float* resid_out;        // optional fp32 residual
  int64_t batch;
  int64_t seq_len;
  int64_t d_model;
  int64_t heads;
  int causal;
  float eps;
  hipStream_t stream;
  const uint8_t* valid_mask = nullptr;  // optional [B, S] token mask, 0 = padded
};
bool layer_small_ok(int64_t seq_len, int64_t d_model, int64_t heads);
// Whether run_layer_small takes this call: the persistent kernel's shapes, or
// the query-split kernel's (which adds head_dim 128) when it pays for the batch.
bool layer_fused_ok(int64_t batch, int64_t seq_len, int64_t d_model, int64_t heads, int x_dtype);
hipError_t run_layer_small(const SmallLayerArgs& a);

// Arguments of the query-split fused kernel (layer_split.hip), one struct of 112 bytes
// passed by value: the HIP runtime's host cost per launch grows with the number of
// kernel arguments and with their size past ~128 bytes (2.9 us for this struct against
// 3.7 us for the same bytes as 16 arguments, and 3.7 us for a 184-byte struct).  Order:
// everything the first transfers need (S, the grid size, x, W_qkv and the parameter
// rows) comes first, in the first 56 bytes of the argument block, which one scalar
// load returns; `nblk` is gridDim.x, passed explicitly so the tile mapping does not
// wait on a second load of the dispatch's hidden arguments.
struct SplitArgs {
  int S, nblk;
  const _Float16* x;
  const _Float16* wqkv;
  const float* bqkv;
  const float* bo;
  const float* g2;
  const float* be2;
  const _Float16* wo;
  const float* g1;    // LN1's elementwise affine (null: none)
  const float* be1;
  void* y;
  float* resid_out;   // optional fp32 residual
  float c2, eps;      // softmax scale * log2(e); LayerNorm epsilon
  const uint8_t* vmask;  // [B, S] token mask (masked variant only)
};
static_assert(sizeof(SplitArgs) == 112, "kernel argument block");
// One call of the query-split kernel resolved once (shape checks, variant, grid,
// arguments); x, y, the token mask and the residual output are set per launch.
struct SplitLaunch {
  const void* fn[2];  // kernel without / with a token mask
  unsigned grid, block;
  SplitArgs args;
};
// Whether run_layer_small would take the query-split kernel for this call.
bool layer_split_takes(const SmallLayerArgs& a);
bool prepare_layer_split(const SmallLayerArgs& a, SplitLaunch* l);
hipError_t launch_layer_split(const SplitLaunch& l, const void* x, const uint8_t* valid_mask, void* y,
                              float* resid_out, hipStream_t stream);

// One transformer block of the fused stack in one launch (the query-split kernel's
// whole-block mode): h = norm1(r) fp16 in, r fp32 in, r_out / out written.
struct BlockArgs {
  const void* h;           // [B*S, D] fp16
  const float* r;          // [B*S, D] fp32 (r_out may equal r)
  const uint8_t* valid_mask;  // optional [B, S], 0 = padded
  const void* w_qkv;       // [3D, D] fp16
  const float* b_qkv;
  const void* w_o;         // [D, D] fp16
  const float* b_o;
  const float* ln2_w;
  const float* ln2_b;
  const void* w1;          // [F, D] fp16
  const float* b1;
  const void* w2;          // [D, F] fp16
  const float* b2;
  const float* lnn_w;      // next norm
  const float* lnn_b;
  float* r_out;            // [B*S, D] fp32
  void* out;               // [B*S, D] out_dtype
  int out_dtype;
  int mask_out;
  int64_t batch;
  int64_t seq_len;
  int64_t d_model;
  int64_t heads;
  int64_t ffn_dim;
  int causal;
  float eps;
  hipStream_t stream;
};
bool block_split_ok(int64_t seq_len, int64_t d_model, int64_t heads, int64_t ffn_dim);
bool block_split_pays(int64_t batch, int64_t seq_len);
hipError_t run_block_split(const BlockArgs& a);

}  // namespace cobra

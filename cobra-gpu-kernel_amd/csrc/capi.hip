// extern "C" entry points (declared in include/cobra_amd.h) and the
// orchestration of the whole attention sublayer.
#include "cobra_amd.h"

#include <atomic>
#include <mutex>
#include <new>

#include "common.hpp"
#include "kernels.hpp"

namespace {

using cobra::kBF16;
using cobra::kF16;
using cobra::kF32;

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool aligned_to(const void* p, int n) { return (reinterpret_cast<uintptr_t>(p) & (uintptr_t)(n - 1)) == 0; }
int dtype_bytes(int dt) { return dt == kF32 ? 4 : 2; }
int64_t round8(int64_t n) { return (n + 7) & ~int64_t(7); }
bool opt_aligned16(const void* p) { return p == nullptr || aligned16(p); }
bool is_dtype(int dt) { return dt == kF16 || dt == kF32; }
bool is_act_dtype(int dt) { return is_dtype(dt) || dt == kBF16; }  // activations that may be bf16
bool is_op_dtype(int dt) { return dt == kF16 || dt == kBF16; }     // 16-bit MFMA operands
int64_t round256(int64_t n) { return (n + 255) & ~int64_t(255); }
int code(hipError_t e) { return static_cast<int>(e); }
constexpr int kBad = static_cast<int>(hipErrorInvalidValue);

constexpr int kEpiAll = COBRA_EPI_GELU | COBRA_EPI_MASK_BRANCH | COBRA_EPI_MASK_RESID | COBRA_EPI_MASK_OUT;
static_assert(COBRA_EPI_GELU == cobra::kEpiGelu && COBRA_EPI_MASK_BRANCH == cobra::kEpiMaskBranch &&
                  COBRA_EPI_MASK_RESID == cobra::kEpiMaskResid && COBRA_EPI_MASK_OUT == cobra::kEpiMaskOut,
              "ABI flag values are the kernels' own");

struct LayerBuffers {
  int64_t h_off, qkv_off, bits_off, total;
};

// Workspace layout of cobra_layer_fwd: h (fp16 [T, D], later reused for the
// attention context), qkv (fp16 [T, 3D]; for D > 128 later reused for the
// out-projection's fp16 branch), and with a token mask the packed key bits
// ([B][ceil(S/64)] u64).
LayerBuffers layer_buffers(int64_t batch, int64_t seq_len, int64_t d, bool masked) {
  const int64_t tokens = batch * seq_len;
  LayerBuffers b{};
  b.h_off = 0;
  b.qkv_off = round256(tokens * d * 2);
  b.bits_off = b.qkv_off + round256(tokens * 3 * d * 2);
  b.total = b.bits_off + (masked ? round256(batch * cobra::mask_words(seq_len) * 8) : 0);
  return b;
}

// LN1's elementwise affine: both parameters, or neither (LayerNorm without affine).
bool ln1_affine_ok(const float* w, const float* b) {
  return (w == nullptr) == (b == nullptr) && opt_aligned16(w) && opt_aligned16(b);
}

bool layer_shape_ok(int64_t batch, int64_t seq_len, int64_t d, int64_t heads) {
  if (batch < 0 || seq_len < 0 || d <= 0 || heads <= 0 || d % heads != 0) return false;
  const int64_t hd = d / heads;
  return hd <= 256 && d <= cobra::kLnMaxD && seq_len <= 0x7fffffff;
}

// Shapes whose head_dim or d_model is not a multiple of 8 run the padded staged plan.
bool layer_needs_pad(int64_t d, int64_t heads) { return d % 8 != 0 || (d / heads) % 8 != 0; }

// Workspace of the padded staged plan: zero-padded weights (each head's rows / columns
// padded from head_dim to hdp = round8(head_dim), d_model to Dp = round8(d_model)), the
// padded activations h / ctx, qkv, the fp32 out-projection branch, the key bits.
struct PadBuffers {
  int64_t hdp, dp, e;  // padded head_dim, d_model, H * hdp
  int64_t wq_off, bq_off, wo_off, bo_off, h_off, qkv_off, r_off, bits_off, total;
};
PadBuffers pad_buffers(int64_t batch, int64_t seq_len, int64_t d, int64_t heads, bool masked) {
  PadBuffers p{};
  const int64_t tokens = batch * seq_len;
  p.hdp = round8(d / heads);
  p.dp = round8(d);
  p.e = heads * p.hdp;
  p.wq_off = 0;
  p.bq_off = p.wq_off + round256(3 * p.e * p.dp * 2);
  p.wo_off = p.bq_off + round256(3 * p.e * 4);
  p.bo_off = p.wo_off + round256(p.dp * p.e * 2);
  p.h_off = p.bo_off + round256(p.dp * 4);
  p.qkv_off = p.h_off + round256(tokens * (p.dp > p.e ? p.dp : p.e) * 2);
  p.r_off = p.qkv_off + round256(tokens * 3 * p.e * 2);
  p.bits_off = p.r_off + round256(tokens * p.dp * 4);
  p.total = p.bits_off + (masked ? round256(batch * cobra::mask_words(seq_len) * 8) : 0);
  return p;
}

}  // namespace

// The workspace of cobra_layer_fwd_noalloc: one copy per device, in the code
// object's zero-initialised data, so it costs no file size and no allocation
// call.  In host code `scratch` names a host-side stand-in, not device memory:
// kernels get the per-device address that hipGetSymbolAddress returns.
static __device__ __align__(256) unsigned char scratch[COBRA_NOALLOC_MAX_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
std::atomic<void*> g_scratch_ptr[kMaxDevices];

// Device address of `scratch` on the current device, looked up with that device
// current (each device holds its own copy) and kept once the lookup succeeds; a failed
// lookup is returned and tried again on the next call.
hipError_t scratch_of_current_device(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (!p) {
      if ((e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch))) != hipSuccess) return e;
      if (!p) return hipErrorInvalidSymbol;
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return hipSuccess;
}

// The padded staged plan (head_dim or d_model not a multiple of 8): the weights are
// laid out zero-padded in the workspace, LN1 writes h padded to Dp columns, the QKV
// GEMM produces q / k / v with every head padded to hdp dimensions, the attention
// runs at head_dim hdp with the true scale (the zero dimensions add nothing to
// q . k and give zero context columns), the out-projection writes its fp32 branch
// [T, Dp] (padded rows zeroed for masked tokens), and LN2 adds x and normalises the
// first D columns.
int layer_fwd_padded(const void* x, int x_dtype, const uint8_t* valid_mask, const void* w_qkv, const float* b_qkv,
                     const void* w_o, const float* b_o, const float* ln1_w, const float* ln1_b, const float* ln2_w,
                     const float* ln2_b, void* y, float* resid_out, void* workspace, int64_t workspace_bytes,
                     int64_t batch, int64_t seq_len, int64_t D, int64_t H, int causal, float eps, hipStream_t s) {
  const bool masked = valid_mask != nullptr;
  const PadBuffers pb = pad_buffers(batch, seq_len, D, H, masked);
  if (!workspace || workspace_bytes < pb.total) return kBad;
  const int64_t T = batch * seq_len;
  if (T == 0) return 0;
  const int64_t hd = D / H, hdp = pb.hdp, Dp = pb.dp, E = pb.e;
  const int op = x_dtype == kBF16 ? kBF16 : kF16;  // MFMA operand type (weights, h, q / k / v, ctx)
  char* ws = static_cast<char*>(workspace);
  void* wq = ws + pb.wq_off;
  float* bq = reinterpret_cast<float*>(ws + pb.bq_off);
  void* wo = ws + pb.wo_off;
  float* bo = reinterpret_cast<float*>(ws + pb.bo_off);
  void* h = ws + pb.h_off;
  void* ctx = h;  // h is dead once the QKV projection has read it
  void* qkv = ws + pb.qkv_off;
  float* r = reinterpret_cast<float*>(ws + pb.r_off);
  uint64_t* bits = masked ? reinterpret_cast<uint64_t*>(ws + pb.bits_off) : nullptr;
  hipError_t e = hipSuccess;
  // W_qkv [3D, D] -> [3E, Dp]: head-padded rows, tail-padded columns; b_qkv likewise.
  cobra::PadArgs p1{w_qkv, wq, 2, D, 3 * E, Dp, hd, hdp, 3 * D, Dp, Dp, D, s};
  cobra::PadArgs p2{b_qkv, bq, 4, 1, 3 * E, 1, hd, hdp, 3 * D, 1, 1, 1, s};
  // W_o [D, D] -> [Dp, E]: tail-padded rows, head-padded columns; b_o tail-padded.
  cobra::PadArgs p3{w_o, wo, 2, D, Dp, E, Dp, Dp, D, hd, hdp, D, s};
  cobra::PadArgs p4{b_o, bo, 4, 1, Dp, 1, Dp, Dp, D, 1, 1, 1, s};
  for (const cobra::PadArgs* pa : {&p1, &p2, &p3, &p4})
    if ((e = cobra::run_pad(*pa)) != hipSuccess) return code(e);
  if (masked && (e = cobra::run_mask_bits(valid_mask, bits, batch, (int)seq_len, s)) != hipSuccess) return code(e);
  cobra::LnArgs ln1{x, x_dtype, nullptr, 0, ln1_w, ln1_b, nullptr, h, op, T, (int)D, eps, s};
  ln1.ldy = Dp;
  if ((e = cobra::run_ln(ln1)) != hipSuccess) return code(e);
  cobra::GemmArgs proj{h, wq, bq, nullptr, op, qkv, op, T, (int)(3 * E), (int)Dp,
                       nullptr, nullptr, nullptr, kF16, eps, s};
  proj.ab_dtype = op;
  if ((e = cobra::run_gemm(proj)) != hipSuccess) return code(e);
  cobra::AttnArgs at{qkv, ctx, batch, (int)seq_len, (int)H, (int)hdp, (float)(1.0 / sqrt((double)hd)),
                     causal ? 1 : 0, s};
  at.key_bits = bits;
  at.dtype = op;
  if ((e = cobra::run_attn(at)) != hipSuccess) return code(e);
  // Padded query rows: the attention output is zeroed before the residual add (TTB:121-122).
  cobra::GemmArgs out{ctx, wo, bo, nullptr, op, r, kF32, T, (int)Dp, (int)E,
                      nullptr, nullptr, nullptr, kF16, eps, s};
  out.ab_dtype = op;
  out.row_mask = valid_mask;
  out.epi = masked ? cobra::kEpiMaskBranch : 0;
  if ((e = cobra::run_gemm(out)) != hipSuccess) return code(e);
  cobra::LnArgs ln2{x, x_dtype, r, 1, ln2_w, ln2_b, resid_out, y, x_dtype, T, (int)D, eps, s};
  ln2.ldb = Dp;
  return code(cobra::run_ln(ln2));
}

// The staged sublayer with bf16 activations and weights (x_dtype kBF16): LN1 into the h
// area (bf16), the QKV GEMM into the qkv area (bf16 q | k | v), the attention into the h
// area, the out-projection with the residual x added in its epilogue storing r in fp32
// (into resid_out, or the qkv area, dead by then: 4 T D of its 6 T D bytes), and LN2 from
// r to y (bf16).  Every product is a bf16 MFMA with fp32 accumulation.
int layer_fwd_bf16(const void* x, const uint8_t* valid_mask, const void* w_qkv, const float* b_qkv, const void* w_o,
                   const float* b_o, const float* ln1_w, const float* ln1_b, const float* ln2_w, const float* ln2_b,
                   void* y, float* resid_out, void* workspace, int64_t workspace_bytes, int64_t batch, int64_t seq_len,
                   int64_t D, int64_t H, int causal, float eps, hipStream_t s) {
  const bool masked = valid_mask != nullptr;
  const LayerBuffers lb = layer_buffers(batch, seq_len, D, masked);
  if (!workspace || workspace_bytes < lb.total) return kBad;
  const int64_t T = batch * seq_len;
  if (T == 0) return 0;
  char* ws = static_cast<char*>(workspace);
  void* h = ws + lb.h_off;
  void* qkv = ws + lb.qkv_off;
  void* ctx = h;  // h is dead once the QKV projection has read it
  uint64_t* bits = masked ? reinterpret_cast<uint64_t*>(ws + lb.bits_off) : nullptr;
  hipError_t e = hipSuccess;
  if (masked && (e = cobra::run_mask_bits(valid_mask, bits, batch, (int)seq_len, s)) != hipSuccess) return code(e);
  const int64_t hd = D / H;
  if (cobra::qkv_attn_head_ok(seq_len, H, hd)) {
    // head_dim 256, S <= 128: as for fp16 -- LN1, the QKV projection fused into the
    // attention (ctx into the qkv area), then the out-projection with LN2 in its epilogue
    // when its grid fits the chip, else the out-projection storing r in fp32 (past ctx in
    // the qkv area, or resid_out) and LN2 reading it.
    cobra::LnArgs ln1{x, kBF16, nullptr, 0, ln1_w, ln1_b, nullptr, h, kBF16, T, (int)D, eps, s};
    if ((e = cobra::run_ln(ln1)) != hipSuccess) return code(e);
    cobra::QkvAttnArgs f{h, w_qkv, b_qkv, qkv, batch, seq_len, H, hd, (float)(1.0 / sqrt((double)hd)),
                         causal ? 1 : 0, bits, s};
    f.dtype = kBF16;
    void* past_ctx = static_cast<char*>(qkv) + round256(T * D * 2);
    if (!resid_out && cobra::gemm_rowln_ok(T, (int)D, (int)D)) {
      f.fill = static_cast<uint64_t*>(past_ctx);
      f.nfill = cobra::gemm_rowln_sync_bytes(T, (int)D) / 8;
      if ((e = cobra::run_qkv_attn_head(f)) != hipSuccess) return code(e);
      cobra::GemmRowLnArgs out{qkv, w_o, b_o, x, ln2_w, ln2_b, y, T, (int)D, (int)D, eps, valid_mask, past_ctx, s};
      out.dtype = kBF16;
      return code(cobra::run_gemm_rowln(out));
    }
    if ((e = cobra::run_qkv_attn_head(f)) != hipSuccess) return code(e);
    float* r = resid_out ? resid_out : static_cast<float*>(past_ctx);
    cobra::GemmArgs out{qkv, w_o, b_o, x, kBF16, r, kF32, T, (int)D, (int)D, nullptr, nullptr, nullptr, kF16, eps, s};
    out.ab_dtype = kBF16;
    out.row_mask = valid_mask;
    out.epi = masked ? cobra::kEpiMaskBranch : 0;
    if ((e = cobra::run_gemm(out)) != hipSuccess) return code(e);
    cobra::LnArgs ln2{r, kF32, nullptr, 0, ln2_w, ln2_b, nullptr, y, kBF16, T, (int)D, eps, s};
    return code(cobra::run_ln(ln2));
  }
  // d_model 64 / 128: LN1 in the QKV projection's prologue and LN2 in the out-projection's
  // epilogue, as for fp16 (three launches); otherwise LN1 -> projection -> attention ->
  // out-projection (r in fp32) -> LN2.
  const bool fused_ln = cobra::ln_gemm_ok(D, kBF16, kBF16);
  if (fused_ln) {
    cobra::LnGemmArgs proj{x, kBF16, ln1_w, ln1_b, w_qkv, b_qkv, qkv, T, (int)(3 * D), D, eps, s};
    proj.ab_dtype = kBF16;
    if ((e = cobra::run_ln_gemm(proj)) != hipSuccess) return code(e);
  } else {
    cobra::LnArgs ln1{x, kBF16, nullptr, 0, ln1_w, ln1_b, nullptr, h, kBF16, T, (int)D, eps, s};
    if ((e = cobra::run_ln(ln1)) != hipSuccess) return code(e);
    cobra::GemmArgs proj{h, w_qkv, b_qkv, nullptr, kBF16, qkv, kBF16, T, (int)(3 * D), (int)D,
                         nullptr, nullptr, nullptr, kF16, eps, s};
    proj.ab_dtype = kBF16;
    if ((e = cobra::run_gemm(proj)) != hipSuccess) return code(e);
  }
  cobra::AttnArgs at{qkv, ctx, batch, (int)seq_len, (int)H, (int)hd, (float)(1.0 / sqrt((double)hd)),
                     causal ? 1 : 0, s};
  at.key_bits = bits;
  at.dtype = kBF16;
  if ((e = cobra::run_attn(at)) != hipSuccess) return code(e);
  // Padded query rows: the attention output is zeroed before the residual add (TTB:121-122).
  if (fused_ln) {
    cobra::GemmArgs out{ctx, w_o, b_o, x, kBF16, resid_out, kF32, T, (int)D, (int)D,
                        ln2_w, ln2_b, y, kBF16, eps, s};
    out.ab_dtype = kBF16;
    out.row_mask = valid_mask;
    out.epi = masked ? cobra::kEpiMaskBranch : 0;
    return code(cobra::run_gemm(out));
  }
  float* r = resid_out ? resid_out : static_cast<float*>(qkv);
  cobra::GemmArgs out{ctx, w_o, b_o, x, kBF16, r, kF32, T, (int)D, (int)D, nullptr, nullptr, nullptr, kF16, eps, s};
  out.ab_dtype = kBF16;
  out.row_mask = valid_mask;
  out.epi = masked ? cobra::kEpiMaskBranch : 0;
  if ((e = cobra::run_gemm(out)) != hipSuccess) return code(e);
  cobra::LnArgs ln2{r, kF32, nullptr, 0, ln2_w, ln2_b, nullptr, y, kBF16, T, (int)D, eps, s};
  return code(cobra::run_ln(ln2));
}

// Out-projection and LN2 of the staged sublayer at d_model > 128: ctx [T, D] fp16 in,
// y out; `spare` is a dead workspace area of at least T * D fp16 and `spare32` one of at
// least T * D fp32, neither overlapping ctx.
int out_proj_ln2(const void* ctx, void* spare, float* spare32, const void* x, int x_dtype,
                 const uint8_t* valid_mask, const void* w_o, const float* b_o, const float* ln2_w,
                 const float* ln2_b, void* y, float* resid_out, int64_t T, int64_t D, float eps, hipStream_t s) {
  const bool masked = valid_mask != nullptr;
  hipError_t e = hipSuccess;
  if (resid_out || x_dtype == kF32) {
    // The out-projection adds x and stores r in fp32 (the reference's split,
    // TTB:1274-1283), LN2 reads it back: into the caller's resid_out when r is an
    // output, and always for fp32 activations, whose branch keeps its fp32 accumulation.
    float* r = resid_out ? resid_out : spare32;
    cobra::GemmArgs out{ctx, w_o, b_o, x, x_dtype, r, kF32, T, (int)D, (int)D,
                        nullptr, nullptr, nullptr, kF16, eps, s};
    out.row_mask = valid_mask;
    out.epi = masked ? cobra::kEpiMaskBranch : 0;
    if ((e = cobra::run_gemm(out)) != hipSuccess) return code(e);
    cobra::LnArgs ln2{r, kF32, nullptr, 0, ln2_w, ln2_b, nullptr, y, x_dtype, T, (int)D, eps, s};
    return code(cobra::run_ln(ln2));
  }
  // fp16 activations, r not requested: the out-projection stores only the branch
  // ctx W_o^T + b_o, in fp16, into the spare area, and LN2 forms r = x + branch in fp32
  // (the reference's _add_ln split, TTB:539): half the bytes of an fp32 r, and no
  // residual read in the GEMM.  The large values of r sit in x, exact in the sum; the
  // branch's rounding is 2^-11 of its own magnitude, so y differs from the resid_out
  // form's by at most that rounding's effect.  (r itself rounded to fp16 would put half
  // an fp16 step of |r| into LN2, amplified by 1/std for inputs with a large mean.)
  cobra::GemmArgs out{ctx, w_o, b_o, nullptr, kF16, spare, kF16, T, (int)D, (int)D,
                      nullptr, nullptr, nullptr, kF16, eps, s};
  out.row_mask = valid_mask;
  out.epi = masked ? cobra::kEpiMaskBranch : 0;
  if ((e = cobra::run_gemm(out)) != hipSuccess) return code(e);
  cobra::LnArgs ln2{x, x_dtype, spare, 0, ln2_w, ln2_b, nullptr, y, x_dtype, T, (int)D, eps, s};
  return code(cobra::run_ln(ln2));
}

}  // namespace

extern "C" {

int cobra_version(void) { return COBRA_ABI_VERSION; }

const char* cobra_error_string(int c) { return hipGetErrorString(static_cast<hipError_t>(c)); }

int cobra_ln_fwd(const void* x, int x_dtype, const void* branch, int branch_dtype, const float* gamma,
                 const float* beta, const uint8_t* row_mask, int mask_flags, float* resid_out, void* y, int y_dtype,
                 int64_t rows, int64_t d, float eps, void* stream) {
  if (rows == 0 && d > 0 && d <= cobra::kLnMaxD && is_act_dtype(x_dtype) && is_act_dtype(y_dtype)) return 0;
  if (!x || !y || !gamma || !beta || !is_act_dtype(x_dtype) || !is_act_dtype(y_dtype)) return kBad;
  if ((mask_flags & ~(COBRA_EPI_MASK_RESID | COBRA_EPI_MASK_OUT)) != 0 || (mask_flags && !row_mask)) return kBad;
  if (branch && !is_dtype(branch_dtype)) return kBad;
  // Element alignment suffices; widths that are multiples of 8 on 16-byte aligned buffers
  // take the vector kernels.
  if (!aligned_to(x, dtype_bytes(x_dtype)) || !aligned_to(y, dtype_bytes(y_dtype)) || !aligned_to(gamma, 4) ||
      !aligned_to(beta, 4) || (branch && !aligned_to(branch, dtype_bytes(branch_dtype))) ||
      (resid_out && !aligned_to(resid_out, 4)))
    return kBad;
  if (d <= 0 || d > cobra::kLnMaxD || rows < 0) return kBad;
  cobra::LnArgs a{x,        x_dtype, branch, branch_dtype == kF32 ? 1 : 0, gamma, beta, resid_out, y, y_dtype,
                  rows,     (int)d,  eps,    static_cast<hipStream_t>(stream)};
  a.row_mask = row_mask;
  a.mask_resid = (mask_flags & COBRA_EPI_MASK_RESID) != 0;
  a.mask_out = (mask_flags & COBRA_EPI_MASK_OUT) != 0;
  return code(cobra::run_ln(a));
}

int cobra_ln_fwd_strided(const void* x, int x_dtype, int64_t ldx, const void* branch, int branch_dtype, int64_t ldb,
                         const float* gamma, const float* beta, const uint8_t* row_mask, int mask_flags,
                         float* resid_out, int64_t ldr, void* y, int y_dtype, int64_t ldy, int64_t rows, int64_t d,
                         float eps, void* stream) {
  if (rows == 0 && d > 0 && d <= cobra::kLnMaxD && is_act_dtype(x_dtype) && is_act_dtype(y_dtype)) return 0;
  if (!x || !y || !gamma || !beta || !is_act_dtype(x_dtype) || !is_act_dtype(y_dtype)) return kBad;
  if ((mask_flags & ~(COBRA_EPI_MASK_RESID | COBRA_EPI_MASK_OUT)) != 0 || (mask_flags && !row_mask)) return kBad;
  if (branch && !is_dtype(branch_dtype)) return kBad;
  if (!aligned_to(x, dtype_bytes(x_dtype)) || !aligned_to(y, dtype_bytes(y_dtype)) || !aligned_to(gamma, 4) ||
      !aligned_to(beta, 4) || (branch && !aligned_to(branch, dtype_bytes(branch_dtype))) ||
      (resid_out && !aligned_to(resid_out, 4)))
    return kBad;
  if (d <= 0 || d > cobra::kLnMaxD || rows < 0) return kBad;
  const int64_t lx = ldx ? ldx : d, lb = ldb ? ldb : d, lr = ldr ? ldr : d, ly = ldy ? ldy : d;
  if (lx < d || lb < d || lr < d || ly < d || ly > cobra::kLnMaxD) return kBad;
  cobra::LnArgs a{x,        x_dtype, branch, branch_dtype == kF32 ? 1 : 0, gamma, beta, resid_out, y, y_dtype,
                  rows,     (int)d,  eps,    static_cast<hipStream_t>(stream)};
  a.row_mask = row_mask;
  a.mask_resid = (mask_flags & COBRA_EPI_MASK_RESID) != 0;
  a.mask_out = (mask_flags & COBRA_EPI_MASK_OUT) != 0;
  a.ldx = lx;
  a.ldb = lb;
  a.ldr = lr;
  a.ldy = ly;
  return code(cobra::run_ln(a));
}

int cobra_linear_fwd(const void* a, const void* w, int ab_dtype, const float* bias, const void* resid, int resid_dtype,
                     const uint8_t* row_mask, int epi, void* c, int c_dtype, int64_t M, int64_t N, int64_t K,
                     void* stream) {
  // resid and c: fp16 or fp32 with fp16 operands, bf16 or fp32 with bf16 operands
  auto out_ok = [&](int dt) { return dt == kF32 || dt == ab_dtype; };
  if (M == 0 && N > 0 && K > 0 && N <= 0x7fffffff && K <= 0x7fffffff && is_op_dtype(ab_dtype) && out_ok(c_dtype))
    return 0;
  if (!a || !w || !c || !is_op_dtype(ab_dtype) || !out_ok(c_dtype) || (resid && !out_ok(resid_dtype))) return kBad;
  if ((epi & ~kEpiAll) != 0 || (epi & COBRA_EPI_MASK_OUT) || ((epi & ~COBRA_EPI_GELU) && !row_mask)) return kBad;
  if (!aligned16(a) || !aligned16(w) || !aligned16(c) || !opt_aligned16(resid) || !opt_aligned16(bias)) return kBad;
  if (M < 0 || N <= 0 || K <= 0 || N > 0x7fffffff || K > 0x7fffffff) return kBad;
  cobra::GemmArgs g{a,       w,       bias,    resid,   resid_dtype, c,   c_dtype,
                    M,       (int)N,  (int)K,  nullptr, nullptr,     nullptr, kF16,
                    1e-5f,   static_cast<hipStream_t>(stream)};
  g.row_mask = row_mask;
  g.epi = epi;
  g.ab_dtype = ab_dtype;
  return code(cobra::run_gemm(g));
}

int cobra_linear_ln_fwd(const void* a, const void* w, const float* bias, const void* resid, int resid_dtype,
                        const uint8_t* row_mask, int epi, float* resid_out, const float* gamma, const float* beta,
                        void* y, int y_dtype, int64_t M, int64_t N, int64_t K, float eps, void* stream) {
  if (M == 0 && N > 0 && N <= 128 && K > 0 && K <= 0x7fffffff && is_dtype(y_dtype)) return 0;
  if (!a || !w || !gamma || !beta || !y || !is_dtype(y_dtype) || (resid && !is_dtype(resid_dtype))) return kBad;
  if ((epi & ~kEpiAll) != 0 || ((epi & ~COBRA_EPI_GELU) && !row_mask)) return kBad;
  if (!aligned16(a) || !aligned16(w) || !aligned16(y) || !opt_aligned16(resid) || !opt_aligned16(resid_out) ||
      !opt_aligned16(bias))
    return kBad;
  if (M < 0 || N <= 0 || N > 128 || K <= 0 || K > 0x7fffffff) return kBad;
  cobra::GemmArgs g{a,     w,      bias,   resid, resid_dtype, resid_out, kF32,
                    M,     (int)N, (int)K, gamma, beta,        y,         y_dtype,
                    eps,   static_cast<hipStream_t>(stream)};
  g.row_mask = row_mask;
  g.epi = epi;
  return code(cobra::run_gemm(g));
}

int cobra_ln_linear_fwd(const void* x, int x_dtype, const float* gamma, const float* beta, const void* w,
                        const float* bias, void* c, int64_t M, int64_t N, int64_t d, float eps, void* stream) {
  if (M == 0 && is_dtype(x_dtype) && cobra::ln_gemm_ok(d, x_dtype) && N > 0 && N <= 0x7fffffff && N % 8 == 0)
    return 0;
  if (!x || !gamma || !beta || !w || !c || !is_dtype(x_dtype)) return kBad;
  if (!aligned16(x) || !aligned16(gamma) || !aligned16(beta) || !aligned16(w) || !aligned16(c) ||
      !opt_aligned16(bias))
    return kBad;
  if (!cobra::ln_gemm_ok(d, x_dtype) || M < 0 || N <= 0 || N > 0x7fffffff || N % 8 != 0) return kBad;
  cobra::LnGemmArgs a{x, x_dtype, gamma, beta, w, bias, c, M, (int)N, d, eps, static_cast<hipStream_t>(stream)};
  return code(cobra::run_ln_gemm(a));
}

int cobra_mask_bits(const uint8_t* mask, uint64_t* key_bits, int64_t batch, int64_t seq_len, void* stream) {
  if ((batch == 0 || seq_len == 0) && batch >= 0 && seq_len >= 0 && seq_len <= 0x7fffffff) return 0;
  if (!mask || !key_bits || (reinterpret_cast<uintptr_t>(key_bits) & 7u) != 0) return kBad;
  if (batch < 0 || seq_len < 0 || seq_len > 0x7fffffff) return kBad;
  return code(cobra::run_mask_bits(mask, key_bits, batch, (int)seq_len, static_cast<hipStream_t>(stream)));
}

int cobra_attn_fwd(const void* qkv, void* ctx, int dtype, const uint64_t* key_bits, int64_t batch, int64_t seq_len,
                   int64_t heads, int64_t head_dim, float scale, int causal, void* stream) {
  if ((batch == 0 || seq_len == 0) && batch >= 0 && seq_len >= 0 && seq_len <= 0x7fffffff && heads > 0 &&
      heads <= 0x7fffffff && head_dim > 0 && head_dim <= 256 && scale > 0.f && is_op_dtype(dtype))
    return 0;
  if (!qkv || !ctx || !aligned16(qkv) || !aligned16(ctx) || !is_op_dtype(dtype)) return kBad;
  if (key_bits && (reinterpret_cast<uintptr_t>(key_bits) & 7u) != 0) return kBad;
  if (batch < 0 || seq_len < 0 || seq_len > 0x7fffffff || heads <= 0 || heads > 0x7fffffff || head_dim <= 0 ||
      head_dim > 256 || !(scale > 0.f))
    return kBad;
  cobra::AttnArgs a{qkv, ctx, batch, (int)seq_len, (int)heads, (int)head_dim, scale, causal ? 1 : 0,
                    static_cast<hipStream_t>(stream)};
  a.key_bits = key_bits;
  a.dtype = dtype;
  return code(cobra::run_attn(a));
}

int64_t cobra_qkv_attn_workspace_bytes(int64_t batch, int64_t seq_len, int64_t heads, int64_t head_dim) {
  if (batch < 0 || seq_len < 0 || heads <= 0 || head_dim <= 0 || head_dim % 8 != 0 || head_dim > 256) return -1;
  if (cobra::qkv_attn_head_ok(seq_len, heads, head_dim)) return 0;  // one fused launch, no q / k / v buffer
  return round256(batch * seq_len * 3 * heads * head_dim * 2);
}

int cobra_qkv_attn_fwd(const void* h, const void* w_qkv, const float* b_qkv, void* ctx, const uint64_t* key_bits,
                       void* workspace, int64_t workspace_bytes, int64_t batch, int64_t seq_len, int64_t heads,
                       int64_t head_dim, float scale, int causal, void* stream) {
  const int64_t need = cobra_qkv_attn_workspace_bytes(batch, seq_len, heads, head_dim);
  if (need < 0 || seq_len > 0x7fffffff || heads > 0x7fffffff || !(scale > 0.f)) return kBad;
  if (batch * seq_len == 0) return 0;
  if (!h || !w_qkv || !ctx || !aligned16(h) || !aligned16(w_qkv) || !aligned16(ctx) || !opt_aligned16(b_qkv))
    return kBad;
  if (key_bits && (reinterpret_cast<uintptr_t>(key_bits) & 7u) != 0) return kBad;
  const int64_t T = batch * seq_len, D = heads * head_dim;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (need == 0) {
    // One launch: the projection inside the attention kernel.  Its workgroups read every
    // h row of their sequence while others write ctx, so the two must not overlap.
    const int64_t hbytes = T * D * 2;
    const char* hc = static_cast<const char*>(h);
    const char* cc = static_cast<const char*>(ctx);
    if (T > 0 && cc < hc + hbytes && hc < cc + hbytes) return kBad;
    if (T == 0) return 0;
    cobra::QkvAttnArgs f{h, w_qkv, b_qkv, ctx, batch, seq_len, heads, head_dim, scale, causal ? 1 : 0,
                         key_bits, s};
    return code(cobra::run_qkv_attn_head(f));
  }
  if (!workspace || !aligned16(workspace) || workspace_bytes < need) return kBad;
  if (T == 0) return 0;
  cobra::GemmArgs proj{h, w_qkv, b_qkv, nullptr, kF16, workspace, kF16, T, (int)(3 * D), (int)D,
                       nullptr, nullptr, nullptr, kF16, 1e-5f, s};
  hipError_t e = cobra::run_gemm(proj);
  if (e != hipSuccess) return code(e);
  cobra::AttnArgs at{workspace, ctx, batch, (int)seq_len, (int)heads, (int)head_dim, scale, causal ? 1 : 0, s};
  at.key_bits = key_bits;
  return code(cobra::run_attn(at));
}

int cobra_layer_plan(int64_t batch, int64_t seq_len, int64_t d_model, int64_t heads, int masked, int x_dtype) {
  if (!layer_shape_ok(batch, seq_len, d_model, heads) || !is_act_dtype(x_dtype)) return -1;
  (void)masked;  // every plan takes a token mask
  if (layer_needs_pad(d_model, heads)) return COBRA_PLAN_PADDED;
  if (x_dtype == kBF16) return COBRA_PLAN_STAGED;  // the fused kernels are fp16-operand
  return cobra::layer_fused_ok(batch, seq_len, d_model, heads, x_dtype) ? COBRA_PLAN_FUSED : COBRA_PLAN_STAGED;
}

int64_t cobra_layer_workspace_bytes(int64_t batch, int64_t seq_len, int64_t d_model, int64_t heads, int masked,
                                    int x_dtype) {
  const int plan = cobra_layer_plan(batch, seq_len, d_model, heads, masked, x_dtype);
  if (plan < 0) return -1;
  if (plan == COBRA_PLAN_PADDED) return pad_buffers(batch, seq_len, d_model, heads, masked != 0).total;
  return plan == COBRA_PLAN_FUSED ? 0 : layer_buffers(batch, seq_len, d_model, masked != 0).total;
}

int cobra_layer_fwd(const void* x, int x_dtype, const uint8_t* valid_mask, const void* w_qkv, const float* b_qkv,
                    const void* w_o, const float* b_o, const float* ln1_w, const float* ln1_b, const float* ln2_w,
                    const float* ln2_b, void* y, float* resid_out, void* workspace, int64_t workspace_bytes,
                    int64_t batch, int64_t seq_len, int64_t d_model, int64_t heads, int causal, float eps,
                    void* stream) {
  const bool masked = valid_mask != nullptr;
  const int plan = cobra_layer_plan(batch, seq_len, d_model, heads, masked, x_dtype);
  if (plan < 0) return kBad;
  if (batch * seq_len == 0) return 0;
  const void* must[] = {x, w_qkv, b_qkv, w_o, b_o, ln2_w, ln2_b, y};
  for (const void* p : must)
    if (!p || !aligned16(p)) return kBad;
  if (!ln1_affine_ok(ln1_w, ln1_b) || !opt_aligned16(resid_out) || !opt_aligned16(workspace)) return kBad;
  const int64_t T = batch * seq_len;
  const int64_t D = d_model;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (plan == COBRA_PLAN_FUSED) {
    if (T == 0) return 0;
    cobra::SmallLayerArgs a{x,     x_dtype, w_qkv, b_qkv, w_o,     b_o,     ln1_w,     ln1_b,   ln2_w, ln2_b,
                            y,     resid_out, batch, seq_len, d_model, heads, causal ? 1 : 0, eps, s};
    a.valid_mask = valid_mask;
    return code(cobra::run_layer_small(a));
  }
  if (plan == COBRA_PLAN_PADDED)
    return layer_fwd_padded(x, x_dtype, valid_mask, w_qkv, b_qkv, w_o, b_o, ln1_w, ln1_b, ln2_w, ln2_b, y, resid_out,
                            workspace, workspace_bytes, batch, seq_len, d_model, heads, causal, eps, s);
  if (x_dtype == kBF16)
    return layer_fwd_bf16(x, valid_mask, w_qkv, b_qkv, w_o, b_o, ln1_w, ln1_b, ln2_w, ln2_b, y, resid_out, workspace,
                          workspace_bytes, batch, seq_len, d_model, heads, causal, eps, s);
  const LayerBuffers lb = layer_buffers(batch, seq_len, D, masked);
  if (!workspace || workspace_bytes < lb.total) return kBad;
  if (T == 0) return 0;
  char* ws = static_cast<char*>(workspace);
  void* h = ws + lb.h_off;
  void* qkv = ws + lb.qkv_off;
  void* ctx = h;  // h is dead once the QKV projection has read it
  uint64_t* bits = masked ? reinterpret_cast<uint64_t*>(ws + lb.bits_off) : nullptr;

  hipError_t e = hipSuccess;
  if (masked && (e = cobra::run_mask_bits(valid_mask, bits, batch, (int)seq_len, s)) != hipSuccess) return code(e);
  const int64_t hd = D / heads;
  if (cobra::qkv_attn_head_ok(seq_len, heads, hd)) {
    // head_dim 256, S <= 128: LN1, then the QKV projection fused into the attention
    // (ctx into the qkv area: the kernel reads every h row while writing ctx), then the
    // out-projection's fp16 branch into the h area (dead by then) and LN2 with x.
    cobra::LnArgs ln1{x, x_dtype, nullptr, 0, ln1_w, ln1_b, nullptr, h, kF16, T, (int)D, eps, s};
    if ((e = cobra::run_ln(ln1)) != hipSuccess) return code(e);
    cobra::QkvAttnArgs f{h, w_qkv, b_qkv, qkv, batch, seq_len, heads, hd, (float)(1.0 / sqrt((double)hd)),
                         causal ? 1 : 0, bits, s};
    if (x_dtype == kF16 && !resid_out && cobra::gemm_rowln_ok(T, (int)D, (int)D)) {
      // fp16 activations, r not requested, the out-projection grid resident at once:
      // LN2 in the out-projection's epilogue (row statistics exchanged between the column
      // tiles of a row block through a sync area past ctx, which the fused QKV kernel
      // marks unwritten).
      void* sync = static_cast<char*>(qkv) + round256(T * D * 2);
      f.fill = static_cast<uint64_t*>(sync);
      f.nfill = cobra::gemm_rowln_sync_bytes(T, (int)D) / 8;
      if ((e = cobra::run_qkv_attn_head(f)) != hipSuccess) return code(e);
      cobra::GemmRowLnArgs out{qkv, w_o, b_o, x, ln2_w, ln2_b, y, T, (int)D, (int)D, eps, valid_mask, sync, s};
      return code(cobra::run_gemm_rowln(out));
    }
    if ((e = cobra::run_qkv_attn_head(f)) != hipSuccess) return code(e);
    // fp32 r (fp32 x): the qkv area past ctx, 4 T D bytes.
    float* r32 = reinterpret_cast<float*>(static_cast<char*>(qkv) + T * D * 2);
    return out_proj_ln2(qkv, h, r32, x, x_dtype, valid_mask, w_o, b_o, ln2_w, ln2_b, y, resid_out, T, D, eps, s);
  }
  if (cobra::ln_gemm_ok(D, x_dtype)) {
    // LN1 in the QKV projection's prologue: h never goes to memory.
    cobra::LnGemmArgs proj{x, x_dtype, ln1_w, ln1_b, w_qkv, b_qkv, qkv, T, (int)(3 * D), D, eps, s};
    if ((e = cobra::run_ln_gemm(proj)) != hipSuccess) return code(e);
  } else {
    cobra::LnArgs ln1{x, x_dtype, nullptr, 0, ln1_w, ln1_b, nullptr, h, kF16, T, (int)D, eps, s};
    if ((e = cobra::run_ln(ln1)) != hipSuccess) return code(e);
    cobra::GemmArgs proj{h, w_qkv, b_qkv, nullptr, kF16, qkv, kF16, T, (int)(3 * D), (int)D,
                         nullptr, nullptr, nullptr, kF16, eps, s};
    if ((e = cobra::run_gemm(proj)) != hipSuccess) return code(e);
  }

  cobra::AttnArgs at{qkv, ctx, batch, (int)seq_len, (int)heads, (int)(D / heads),
                     (float)(1.0 / sqrt((double)(D / heads))), causal ? 1 : 0, s};
  at.key_bits = bits;
  if ((e = cobra::run_attn(at)) != hipSuccess) return code(e);

  // Padded query rows: the attention output is zeroed before the residual add
  // (TTB:121-122), so r = x there.
  if (D <= 128) {
    cobra::GemmArgs out{ctx, w_o, b_o, x, x_dtype, resid_out, kF32, T, (int)D, (int)D,
                        ln2_w, ln2_b, y, x_dtype, eps, s};
    out.row_mask = valid_mask;
    out.epi = masked ? cobra::kEpiMaskBranch : 0;
    return code(cobra::run_gemm(out));
  }
  return out_proj_ln2(ctx, qkv, static_cast<float*>(qkv), x, x_dtype, valid_mask, w_o, b_o, ln2_w, ln2_b, y,
                      resid_out, T, D, eps, s);
}


struct cobra_layer_launch {
  int x_dtype, masked, causal;
  const void* w_qkv;
  const float *b_qkv, *b_o, *ln1_w, *ln1_b, *ln2_w, *ln2_b;
  const void* w_o;
  void* workspace;
  int64_t workspace_bytes, batch, seq_len, d_model, heads;
  float eps;
  // The query-split kernel's launch resolved at bind time (plan, variant, grid and
  // arguments), so a run costs one hipLaunchKernel: at the small shapes that kernel
  // takes ~7 us and the host's launch path is most of a forward's host time.
  bool split;
  cobra::SplitLaunch sl;
};

cobra_layer_launch* cobra_layer_bind(int x_dtype, int masked, const void* w_qkv, const float* b_qkv, const void* w_o,
                                     const float* b_o, const float* ln1_w, const float* ln1_b, const float* ln2_w,
                                     const float* ln2_b, void* workspace, int64_t workspace_bytes, int64_t batch,
                                     int64_t seq_len, int64_t d_model, int64_t heads, int causal, float eps) {
  const int plan = cobra_layer_plan(batch, seq_len, d_model, heads, masked, x_dtype);
  if (plan < 0) return nullptr;
  const void* must[] = {w_qkv, b_qkv, w_o, b_o, ln2_w, ln2_b};
  for (const void* p : must)
    if (!p || !aligned16(p)) return nullptr;
  if (!ln1_affine_ok(ln1_w, ln1_b) || !opt_aligned16(workspace)) return nullptr;
  const int64_t need = cobra_layer_workspace_bytes(batch, seq_len, d_model, heads, masked, x_dtype);
  if (need > 0 && (!workspace || workspace_bytes < need)) return nullptr;
  auto* h = new (std::nothrow) cobra_layer_launch;
  if (!h) return nullptr;
  *h = cobra_layer_launch{x_dtype, masked ? 1 : 0, causal ? 1 : 0, w_qkv, b_qkv, b_o, ln1_w, ln1_b, ln2_w, ln2_b,
                          w_o, workspace, workspace_bytes, batch, seq_len, d_model, heads, eps, false, {}};
  if (plan == COBRA_PLAN_FUSED && batch > 0) {
    cobra::SmallLayerArgs a{nullptr, x_dtype, w_qkv,   b_qkv,   w_o,   b_o,          ln1_w, ln1_b, ln2_w, ln2_b,
                            nullptr, nullptr, batch, seq_len, d_model, heads, causal ? 1 : 0, eps, nullptr};
    h->split = cobra::prepare_layer_split(a, &h->sl);
  }
  return h;
}

int cobra_layer_run(const cobra_layer_launch* h, const void* x, const uint8_t* valid_mask, void* y, float* resid_out,
                    void* stream) {
  if (!h || (valid_mask && !h->masked)) return kBad;
  if (h->batch * h->seq_len == 0) return 0;
  if (h->split) {
    if (!x || !aligned16(x) || !y || !aligned16(y) || !opt_aligned16(resid_out)) return kBad;
    return code(cobra::launch_layer_split(h->sl, x, valid_mask, y, resid_out, static_cast<hipStream_t>(stream)));
  }
  return cobra_layer_fwd(x, h->x_dtype, valid_mask, h->w_qkv, h->b_qkv, h->w_o, h->b_o, h->ln1_w, h->ln1_b, h->ln2_w,
                         h->ln2_b, y, resid_out, h->workspace, h->workspace_bytes, h->batch, h->seq_len, h->d_model,
                         h->heads, h->causal, h->eps, stream);
}

void cobra_layer_unbind(cobra_layer_launch* h) { delete h; }

int cobra_layer_fwd_noalloc(const void* x, int x_dtype, const uint8_t* valid_mask, const void* w_qkv,
                            const float* b_qkv, const void* w_o, const float* b_o, const float* ln1_w,
                            const float* ln1_b, const float* ln2_w, const float* ln2_b, void* y, float* resid_out,
                            int64_t batch, int64_t seq_len, int64_t d_model, int64_t heads, int causal, float eps,
                            void* stream) {
  const int64_t need =
      cobra_layer_workspace_bytes(batch, seq_len, d_model, heads, valid_mask != nullptr, x_dtype);
  if (need < 0 || need > COBRA_NOALLOC_MAX_BYTES) return kBad;
  if (batch * seq_len == 0) return 0;
  void* ws = nullptr;
  if (need > 0) {
    int cur = -1, sdev = -1;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) return code(e);
    if (stream) {
      if ((e = hipStreamGetDevice(static_cast<hipStream_t>(stream), &sdev)) != hipSuccess) return code(e);
      if (sdev != cur) return kBad;
    }
    if ((e = scratch_of_current_device(&ws)) != hipSuccess) return code(e);
  }
  return cobra_layer_fwd(x, x_dtype, valid_mask, w_qkv, b_qkv, w_o, b_o, ln1_w, ln1_b, ln2_w, ln2_b, y, resid_out,
                         ws, need, batch, seq_len, d_model, heads, causal, eps, stream);
}

int cobra_block_plan(int64_t batch, int64_t seq_len, int64_t d_model, int64_t heads, int64_t ffn_dim) {
  if (batch < 0 || !cobra::block_split_ok(seq_len, d_model, heads, ffn_dim)) return -1;
  return cobra::block_split_pays(batch, seq_len) ? 1 : 0;
}

int cobra_block_fwd(const void* h, const float* r, const uint8_t* valid_mask, const void* w_qkv, const float* b_qkv,
                    const void* w_o, const float* b_o, const float* ln2_w, const float* ln2_b, const void* w1,
                    const float* b1, const void* w2, const float* b2, const float* lnn_w, const float* lnn_b,
                    float* r_out, void* out, int out_dtype, int mask_out, int64_t batch, int64_t seq_len,
                    int64_t d_model, int64_t heads, int64_t ffn_dim, int causal, float eps, void* stream) {
  if (cobra_block_plan(batch, seq_len, d_model, heads, ffn_dim) < 0 || !is_dtype(out_dtype)) return kBad;
  if (batch * seq_len == 0) return 0;
  const void* must[] = {h, r, w_qkv, b_qkv, w_o, b_o, ln2_w, ln2_b, w1, b1, w2, b2, lnn_w, lnn_b, r_out, out};
  for (const void* p : must)
    if (!p || !aligned16(p)) return kBad;
  if (mask_out && !valid_mask) return kBad;
  // out must not overlap h (every workgroup of a sequence reads all of its h rows) or r.
  const int64_t T = batch * seq_len;
  auto overlaps = [](const void* a, int64_t na, const void* b, int64_t nb) {
    const char* pa = static_cast<const char*>(a);
    const char* pb = static_cast<const char*>(b);
    return pa < pb + nb && pb < pa + na;
  };
  const int64_t hb = T * d_model * 2, rb = T * d_model * 4, ob = T * d_model * dtype_bytes(out_dtype);
  if (overlaps(out, ob, h, hb) || overlaps(out, ob, r, rb) || overlaps(out, ob, r_out, rb) ||
      overlaps(r_out, rb, h, hb) || (r_out != r && overlaps(r_out, rb, r, rb)))
    return kBad;
  cobra::BlockArgs a{h,     r,     valid_mask, w_qkv, b_qkv,    w_o,     b_o,   ln2_w, ln2_b,
                     w1,    b1,    w2,         b2,    lnn_w,    lnn_b,   r_out, out,   out_dtype,
                     mask_out ? 1 : 0, batch, seq_len, d_model, heads, ffn_dim, causal ? 1 : 0, eps,
                     static_cast<hipStream_t>(stream)};
  return code(cobra::run_block_split(a));
}

}  // extern "C"

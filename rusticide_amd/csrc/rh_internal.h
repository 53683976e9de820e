// rh_internal.h -- types shared by the C ABI (api.hip) and the kernel
// launchers (quantize.hip, gemv.hip, gemm.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <string>
#include <vector>

#include "../../include/rusticide_hip.h"

namespace rh {

constexpr int kMaxJobs = 8;       // matrices one GEMV launch can serve
constexpr int kMaxTokens = 8;     // tokens one GEMV launch can serve
constexpr size_t kMaxFusedTokens = 4;  // tokens a quantize-fused k-quant launch serves
constexpr size_t kPad = 256;      // bytes of slack after every device matrix

// The quantized activations of one batch on the device, laid out per token:
// quants [tokens][qstride] i8, scales/sums [tokens][bstride] per 32-block,
// sums16 [tokens][2*bstride] per 16-block (Q6_K's -32 offset), and for the
// Row kind the one divisor per token.
struct Q8Dev {
  int8_t* quants = nullptr;
  float* scales = nullptr;
  int32_t* sums = nullptr;
  int32_t* sums16 = nullptr;
  size_t qstride = 0;   // bytes of quants per token
  size_t bstride = 0;   // 32-blocks reserved per token
  size_t n_blocks = 0;  // 32-blocks actually quantized per token
};

// One matrix of a grouped launch.
struct GemvJob {
  // Q4_K / Q6_K: the matrix in the unit layout (rh_device.h); I2_S: rows of
  // `stride` bytes; dense: f32 rows
  const uint8_t* w;
  // A second matrix of w's shape (the up projection beside the gate one):
  // the norm-fused k-quant launch then writes silu(w x) * (w2 x) to out
  // instead of w x.
  const uint8_t* w2;
  float* out;           // out[row * tokens + token] (token-major: out[token * rows + row])
  size_t out_len;
  uint32_t stride;      // bytes between rows (I2_S, dense; a matrix stays below 4 GiB)
  uint32_t rows;        // rows to compute (already bounded by out_len)
  uint32_t nb;          // blocks per row both operands cover
  float scale;          // I2_S tensor scale
  uint32_t wg_begin;    // first workgroup of this job in the grid
  // 0: a workgroup's rows are contiguous. c > 0: iteration k of workgroup w
  // takes the 2^(c-1)-row chunk k * nwg + w, so at any moment the grid reads
  // one window of the matrix (the launcher sets it only when the rows tile
  // the grid exactly).
  uint32_t il = 0;
  uint32_t ub = 0;      // the matrix's blocks per row: block (r, b) is unit block r * ub + b
  uint32_t tmajor = 0;  // k-quant GEMM only: 1 stores out token-major
};
// 64 bytes: every launch's kernel arguments hold kMaxJobs of these
static_assert(sizeof(GemvJob) == 64, "GemvJob packs into 64 bytes");

struct GemvJobs {
  GemvJob j[kMaxJobs];
  uint32_t n;
};

// The residual add and RMSNorm a fused one-token k-quant GEMV launch applies
// to its activation before quantizing it: v = h + delta (h when delta is
// null), x = (v / sqrt(mean(v*v) + eps)) * weight, the sum of squares in
// element order (transformer/src/norm.rs:10-14, portable/norm.rs:8-14). The
// launch's first workgroup writes v to hidden_out when that is set.
struct PickPart;  // rh_device.h
struct NormIn {
  const float* delta = nullptr;
  const float* weight = nullptr;
  float eps = 0.0f;
  float* hidden_out = nullptr;
  uint32_t lds_offset = 0;  // filled by the launcher
  // One job of one-token rows: each workgroup also writes the greedy pick's
  // partial over its rows to pick[workgroup] (a device array), and the
  // launcher stores the workgroup count in *grid_out (host memory).
  PickPart* pick = nullptr;
  uint32_t* grid_out = nullptr;
};

// Kernel choices, read from the environment by the first rh_init (and by
// each rh_reload_tuning) instead of on every launch; each read publishes an
// immutable snapshot, so a launch on another thread sees one whole snapshot. Every choice gives the same
// bits; the switches exist to test and time one kernel against another.
struct Tuning {
  // RUSTICIDE_HIP_GEMV: 0 the quantize-fused decode kernels (decode-sized
  // batches), 1 "lds" (a quantize launch, then kernels that read the
  // quantized activation)
  int gemv = 0;
  int gemv_ni = 0;         // RUSTICIDE_HIP_GEMV_NI=1|2|4|8: blocks per team
  bool interleave = true;  // RUSTICIDE_HIP_GEMV_IL=0: contiguous rows
  int norm_ni = 0;         // RUSTICIDE_HIP_NORM_NI=2|4
  int kq_nt = 0;           // RUSTICIDE_HIP_KQ_NT=256|512: threads per one-token k-quant workgroup
  int norm_nt = 0;         // RUSTICIDE_HIP_NORM_NT=256|512: the same, norm-fused launches
  bool kq_fix = true;      // RUSTICIDE_HIP_KQ_FIX=0: the general block walk only
  bool kq_balance = true;  // RUSTICIDE_HIP_KQ_BALANCE=0: no one-workgroup-per-CU reshaping
  bool kq_onepass = true;  // RUSTICIDE_HIP_KQ_ONEPASS=0: no 768/1024-lane one-round quantization
  int i2s_groups = 0;      // RUSTICIDE_HIP_I2S_GROUPS=1|2|4 (two-token kernel)
  int i2s_lpr = 0;         // RUSTICIDE_HIP_I2S_LPR=8|16|32|64: lanes per row, one token
  int i2s_nt = 0;          // RUSTICIDE_HIP_I2S_NT=256|512|1024: threads per workgroup, one token
  bool i2s_one = true;     // RUSTICIDE_HIP_I2S_ONE=0: one token on the two-token kernel
  int gemm_bn = 0;         // RUSTICIDE_HIP_GEMM_BN=32|64: tokens a GEMM workgroup
  bool gemm_split = true;  // RUSTICIDE_HIP_GEMM_SPLIT=0
  bool gemm_fixup = true;  // RUSTICIDE_HIP_GEMM_FIXUP=0: a split GEMM's planes summed by gemm_combine_kernel
  bool attn_lds = true;    // RUSTICIDE_HIP_ATTN_LDS=0: the tiled attention step only
};
const Tuning& tuning();
void load_tuning();  // publish a fresh snapshot from the environment
void init_tuning();  // load_tuning once per process

// Launchers (stream-ordered; they return the launch status).
hipError_t launch_quantize_super(const float* x, size_t width, size_t tokens, const Q8Dev& q,
                                 hipStream_t s);
hipError_t launch_quantize_row(const float* x, size_t width, size_t tokens, const Q8Dev& q,
                               hipStream_t s);

// Bytes of a k-quant matrix of rows x nb blocks in the unit layout
// (rh_device.h): whole groups of 16 blocks.
size_t units_bytes(uint32_t type_id, size_t rows, size_t nb);

// A split launch's planes left for the caller to sum (SplitOut.planes == 0:
// the launch was not split and stored its outputs itself). Plane p holds, at
// [token][rows_pad] over the launch's row tiles (a job's rows from its
// wg_begin * 128 on), segment 0's in-order sum for p = 0 and block
// seg_len + p - 1's term after it; the outputs are plane 0 plus planes 1..
// in order, one addition at a time.
struct SplitOut {
  const float* terms = nullptr;
  uint32_t planes = 0, rows_pad = 0;
};
// Grouped GEMV for one format: tokens [t0, t0+tn) of `tokens` total.
hipError_t launch_gemv(uint32_t type_id, const GemvJobs& jobs, const Q8Dev& q, const float* x,
                       size_t width, size_t tokens, size_t t0, size_t tn, hipStream_t s,
                       int32_t* raw_i32);
size_t gemv_max_tokens(uint32_t type_id, uint32_t nb);
// Single-launch decode GEMV: every workgroup quantizes the f32 activation of
// its tokens into LDS itself (the same arithmetic as the quantize kernels).
// gemv_fused_ok says whether a launch of tn tokens of `width` values fits it
// (k-quants: tn <= kMaxFusedTokens; I2_S: tn <= 2, width <= 8192).
bool gemv_fused_ok(uint32_t type_id, size_t width, size_t tn);
// With `norm`, x is the hidden state h of one token and the k-quant kernels
// form the normalized activation themselves (norm_fusable says when).
hipError_t launch_gemv_fused(uint32_t type_id, const GemvJobs& jobs, const float* x, size_t width,
                             size_t tokens, size_t t0, size_t tn, hipStream_t s, int32_t* raw,
                             const NormIn* norm = nullptr);
bool norm_fusable(uint32_t type_id, size_t width, uint32_t nbmax);
// Prefill GEMM on MFMA for the k-quants (Q4_K, Q6_K): every row of every job
// against all `tokens` tokens of the quantized activation q, bit-identical to
// the GEMV kernels (and so to the CPU path).
// The float scratch a k-quant GEMM launch over `jobs` needs when it splits K
// across workgroups (0: it does not split). launch_gemm splits only when
// `terms` holds that many bytes; without it the launch runs unsplit.
size_t gemm_split_bytes(uint32_t type_id, const GemvJobs& jobs, size_t tokens);
// Compute units of the current device when first asked (256 if the query
// fails); the launch shapes are sized by it.
int device_cus();
// rh_matmul_batch_device for k-quant jobs on an activation already quantized
// to Q8_K in `q` (width / 256 super-blocks for each of `tokens` tokens).
// token_major: the outputs are stored out[token * rows + row] (same values);
// only the GEMM path stores so, so tokens must be at least rh_gemm_min_tokens().
// defer (token_major only): a split launch leaves its planes there for the
// caller (see launch_gemm); one k-quant job.
rh_status matmul_q8_device(rh_ctx* ctx, const Q8Dev& q, size_t width, size_t tokens, const rh_job* jobs,
                           size_t n_jobs, hipStream_t s, bool token_major = false, SplitOut* defer = nullptr);
// Whether a k-quant GEMM can address a batch: the quantized activation's
// offsets (tokens x qstride bytes) are 32-bit.
bool gemm_fits(size_t tokens, size_t qstride);
// Tiles (row tiles x token tiles) of a split k-quant GEMM launch whose
// last-arriving segment sums the planes itself: `counters` of launch_gemm
// holds this many u32, all zero between launches (each launch leaves them
// so); larger launches, and batches whose token count is not a multiple of
// 4, sum them in a gemm_combine_kernel launch. Launches that share the
// counters must not overlap (one stream).
constexpr uint32_t kFixupTiles = 16384;
// With defer, a split launch stores its planes token-major and leaves them
// in *defer instead of combining them.
hipError_t launch_gemm(uint32_t type_id, const GemvJobs& jobs, const Q8Dev& q, size_t tokens, float* terms,
                       hipStream_t s, SplitOut* defer = nullptr, uint32_t* counters = nullptr);
// Prefill GEMM on int8 MFMA for I2_S against the I8_S activation q; with
// `raw` the i32 dots go there instead of the scaled outputs.
hipError_t launch_gemm_i2s(const GemvJobs& jobs, const Q8Dev& q, size_t tokens, int32_t* raw, hipStream_t s);

}  // namespace rh

struct rh_ctx;
struct rh_matrix;

namespace rh {

// Internal views of the ABI's opaque handles (api.hip).
int ctx_device(const rh_ctx* ctx);
// Changes whenever the context's scratch buffers move (a graph that captured
// their addresses is stale from then on).
uint64_t ctx_scratch_generation(const rh_ctx* ctx);
// Records `msg` as the context's rh_last_error and returns `st`.
rh_status set_last_error(rh_ctx* ctx, rh_status st, const std::string& msg);
const uint8_t* matrix_data(const rh_matrix* m);
// What locates a row: its byte stride for f32 rows, its block count for a
// k-quant matrix in the unit layout.
size_t matrix_pitch(const rh_matrix* m);

// A matrix checked and allocated on the device (Matrix::load_on's checks,
// model/src/weights.rs:53-98) whose image is not uploaded yet: `src` holds
// its rows back to back (`widened` owns them for an F16 source).
struct PendingUpload {
  rh_matrix* m = nullptr;
  const uint8_t* src = nullptr;
  std::vector<float> widened;
};
rh_status matrix_prepare(rh_ctx* ctx, uint32_t type_id, const void* data, size_t len, size_t rows, size_t cols,
                         PendingUpload* out);
// Uploads the images of `n` prepared matrices (rows at their HBM stride,
// zeros elsewhere) and waits for the copies. On failure the matrices stay
// allocated for the caller to free.
rh_status matrix_upload(rh_ctx* ctx, PendingUpload* p, size_t n);

// Row `row` of matrix data `m` (pitch: matrix_pitch), its first nb blocks
// dequantized into out (at most out_len values).
hipError_t launch_dequantize_row(uint32_t type_id, const uint8_t* m, size_t pitch, uint32_t row, uint32_t nb,
                                 float scale, float* out, size_t out_len, hipStream_t s);

// rh_matmul_batch_device for one token whose activation the k-quant
// kernels form themselves from the hidden state: normalize(hidden + delta) *
// weight (NormIn). Every job must be Q4_K or Q6_K with cols = width and
// norm_fusable; the caller checks that once.
rh_status matmul_norm_device(rh_ctx* ctx, const float* hidden, const NormIn& norm, size_t width, const rh_job* jobs,
                             size_t n_jobs, hipStream_t s);
// The feed-forward's first half for one token in one launch:
// out[r] = silu(gate_r . x) * (up_r . x) for rows r < rows, x the normalized
// activation as above (feed_forward.rs:51-66). gate and up must be k-quant
// matrices of one type, shape and stride (gate_up_pairable says when).
bool gate_up_pairable(const rh_matrix* gate, const rh_matrix* up, size_t width);
rh_status matmul_norm_silu_device(rh_ctx* ctx, const float* hidden, const NormIn& norm, size_t width,
                                  const rh_matrix* gate, const rh_matrix* up, float* out, size_t rows, hipStream_t s);

}  // namespace rh

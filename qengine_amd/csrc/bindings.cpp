// torch bindings for qengine_amd._C: the reference's qengine._C attention ops with the same
// Python signatures and the same validation contract (reference csrc/bindings.cpp:1-30,147-183).
// Every op writes into caller-provided tensors (no allocation), enqueues on the current HIP stream
// and never syncs, so it can be captured in a hipGraph. Row-batched arguments are 2-D views
// [n, width] with stride(1) == 1 and any row stride (a 1-D tensor counts as one row).
//
// Each op is a thin shell over the C ABI in include/qe_attn.h. Launch errors are raised as
// RuntimeError; the reference dropped them (csrc/common.cuh:45).
//
// The _check_* functions run the same validation without the device requirement and without a
// launch, so the contract can be exercised on a machine without a GPU.
#include <cmath>
#include <limits>

#include <torch/extension.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>

#include "qe_attn.h"
#include "qe_gdn.h"
#include "qe_gemv.h"
#include "qe_step.h"

namespace {
const auto BF = torch::kBFloat16;
const auto I32 = torch::kInt32;
const auto F32 = torch::kFloat32;
constexpr int HD = 256;

hipStream_t stream_of(const torch::Tensor& t) {
  return c10::hip::getCurrentHIPStream(t.device().index()).stream();
}

void chk(const torch::Tensor& t, torch::ScalarType dt, const char* name, bool dev) {
  if (dev) TORCH_CHECK(t.is_cuda(), name, " must be a GPU tensor");
  TORCH_CHECK(t.scalar_type() == dt, name, " has wrong dtype ", t.scalar_type());
  TORCH_CHECK(t.is_contiguous(), name, " must be contiguous");
}

// Row view: (rows, width, row stride).
struct Rows {
  int n;
  long w;
  long ld;
};
Rows rows(const torch::Tensor& t, torch::ScalarType dt, const char* name, bool dev) {
  TORCH_CHECK((!dev || t.is_cuda()) && t.scalar_type() == dt, name, ": wrong device/dtype");
  if (t.dim() == 1) {
    TORCH_CHECK(t.stride(0) == 1, name, " not contiguous");
    return {1, (long)t.size(0), (long)t.size(0)};
  }
  TORCH_CHECK(t.dim() == 2 && t.stride(1) == 1, name, " must be [n, w] with unit inner stride");
  return {(int)t.size(0), (long)t.size(1), (long)t.stride(0)};
}

void chk16(const torch::Tensor& t, long ld, const char* name) {
  TORCH_CHECK(reinterpret_cast<uintptr_t>(t.data_ptr()) % 16 == 0 && ld % 8 == 0, name,
              " must be 16-byte aligned rows");
}

// The fp8 KV cache: E4M3FN codes, as torch.float8_e4m3fn or raw uint8 bytes.
void chk_kv8(const torch::Tensor& t, const char* name, bool dev) {
  if (dev) TORCH_CHECK(t.is_cuda(), name, " must be a GPU tensor");
  TORCH_CHECK(t.scalar_type() == torch::kFloat8_e4m3fn || t.scalar_type() == torch::kByte, name,
              " must be float8_e4m3fn (or uint8 codes), got ", t.scalar_type());
  TORCH_CHECK(t.is_contiguous(), name, " must be contiguous");
}

void chk_pos(const torch::Tensor& pos, bool dev) {
  TORCH_CHECK((!dev || pos.is_cuda()) && pos.scalar_type() == I32 && pos.numel() >= 1,
              "pos must be an int32 GPU tensor with at least one element");
}

void raise_on(hipError_t e, const char* what) {
  TORCH_CHECK(e == hipSuccess, what, " failed: ", hipGetErrorString(e));
}

struct PrepArgs {
  int n, Hq, Hkv, max_len, rd;
  long ldp;
};

PrepArgs parse_prep(const torch::Tensor& qg, const torch::Tensor& k, const torch::Tensor& v,
                    const torch::Tensor& qnw, const torch::Tensor& knw,
                    const torch::Tensor& inv_freq, const torch::Tensor& pos,
                    const torch::Tensor& q_out, const torch::Tensor& kc, const torch::Tensor& vc,
                    bool dev, int max_rows = 8, bool kv8 = false) {
  auto QG = rows(qg, BF, "qg", dev), K = rows(k, BF, "k", dev), V = rows(v, BF, "v", dev);
  auto QO = rows(q_out, BF, "q_out", dev);
  TORCH_CHECK(QG.ld == K.ld && QG.ld == V.ld, "qg/k/v must share a row stride");
  chk(qnw, BF, "qnw", dev);
  chk(knw, BF, "knw", dev);
  if (kv8) {
    chk_kv8(kc, "kc", dev);
    chk_kv8(vc, "vc", dev);
  } else {
    chk(kc, BF, "kc", dev);
    chk(vc, BF, "vc", dev);
  }
  chk(inv_freq, F32, "inv_freq", dev);
  chk_pos(pos, dev);
  TORCH_CHECK(kc.dim() == 3 && kc.size(2) == HD, "head_dim 256 only");
  const int n = QG.n, Hkv = kc.size(0), max_len = kc.size(1), Hq = QO.w / HD;
  TORCH_CHECK(n >= 1 && n <= max_rows && K.n == n && V.n == n && QO.n == n && QO.ld == QO.w,
              "prep takes 1..", max_rows, " rows, equal in every argument, and contiguous q_out rows");
  TORCH_CHECK(QO.w == (long)Hq * HD, "q_out width must be Hq*256");
  TORCH_CHECK(Hq >= 1 && QG.w == (long)Hq * 2 * HD && K.w == (long)Hkv * HD &&
                  V.w == (long)Hkv * HD,
              "row widths must be qg = Hq*512, k = v = Hkv*256");
  TORCH_CHECK(vc.sizes() == kc.sizes() && qnw.numel() == HD && knw.numel() == HD,
              "vc must match kc; qnw/knw must have 256 elements");
  const int rd = inv_freq.numel() * 2;
  TORCH_CHECK(rd <= HD, "rotary dims (2 * inv_freq.numel()) must be <= 256");
  return {n, Hq, Hkv, max_len, rd, QG.ld};
}

struct DecodeArgs {
  int n, Hq, Hkv, max_len, NS;
  long ldp, ldo;
};

DecodeArgs parse_decode(const torch::Tensor& q, const torch::Tensor& kc, const torch::Tensor& vc,
                        const torch::Tensor& pos, const torch::Tensor& qg,
                        const torch::Tensor& part_o, const torch::Tensor& part_ml,
                        const torch::Tensor& out, bool dev, bool kv8 = false) {
  auto Qr = rows(q, BF, "q", dev), QG = rows(qg, BF, "qg", dev), O = rows(out, BF, "out", dev);
  if (kv8) {
    chk_kv8(kc, "kc", dev);
    chk_kv8(vc, "vc", dev);
  } else {
    chk(kc, BF, "kc", dev);
    chk(vc, BF, "vc", dev);
  }
  chk(part_o, F32, "part_o", dev);
  chk(part_ml, F32, "part_ml", dev);
  chk_pos(pos, dev);
  chk16(q, Qr.ld, "q");
  chk16(kc, HD, "kc");
  chk16(vc, HD, "vc");
  TORCH_CHECK(kc.dim() == 3 && kc.size(2) == HD && vc.sizes() == kc.sizes(),
              "kc/vc must be [Hkv, max_len, 256] with equal sizes");
  const int n = Qr.n, Hq = Qr.w / HD, Hkv = kc.size(0), max_len = kc.size(1);
  TORCH_CHECK(Hq >= 1 && Qr.ld == Qr.w && QG.n == n && O.n == n && Hq % Hkv == 0,
              "q rows must be contiguous, rows must agree and Hq % Hkv == 0");
  TORCH_CHECK(Qr.w == (long)Hq * HD, "q width must be Hq*256");
  TORCH_CHECK(part_o.dim() == 4 && part_o.size(0) >= n && part_o.size(1) == Hq &&
                  part_o.size(3) == HD,
              "part_o must be [>=n, Hq, NS, 256]");
  const int NS = part_o.size(2);
  TORCH_CHECK(part_ml.numel() == part_o.size(0) * Hq * NS * 2 && O.w == (long)Hq * HD &&
                  QG.w == (long)Hq * 2 * HD,
              "part_ml must be [>=n, Hq, NS, 2]; out width Hq*256; qg width Hq*512");
  TORCH_CHECK(n >= 1 && n <= 65535, "decode takes 1..65535 rows");
  TORCH_CHECK(NS >= 1, "part_o needs at least one split");
  return {n, Hq, Hkv, max_len, NS, QG.ld, O.ld};
}
}  // namespace

// pos: int32 tensor whose element 0 is the position of row 0.
void attn_prep(torch::Tensor qg, torch::Tensor k, torch::Tensor v, torch::Tensor qnw,
               torch::Tensor knw, torch::Tensor inv_freq, torch::Tensor pos, torch::Tensor q_out,
               torch::Tensor kc, torch::Tensor vc, double eps) {
  const auto a = parse_prep(qg, k, v, qnw, knw, inv_freq, pos, q_out, kc, vc, true);
  const c10::DeviceGuard guard(qg.device());
  raise_on(qe_attn_prep(qg.data_ptr(), k.data_ptr(), v.data_ptr(), a.ldp, qnw.data_ptr(),
                        knw.data_ptr(), inv_freq.data_ptr<float>(), pos.data_ptr<int>(),
                        q_out.data_ptr(), kc.data_ptr(), vc.data_ptr(), a.n, a.Hq, a.Hkv,
                        a.max_len, a.rd, (float)eps, stream_of(qg)),
           "qe_attn_prep");
}

// attn_prep for a prefill chunk: the same op without the 8-row limit (rows up to 65535).
void attn_prep_chunk(torch::Tensor qg, torch::Tensor k, torch::Tensor v, torch::Tensor qnw,
                     torch::Tensor knw, torch::Tensor inv_freq, torch::Tensor pos,
                     torch::Tensor q_out, torch::Tensor kc, torch::Tensor vc, double eps) {
  const auto a = parse_prep(qg, k, v, qnw, knw, inv_freq, pos, q_out, kc, vc, true, 65535);
  const c10::DeviceGuard guard(qg.device());
  raise_on(qe_attn_prep(qg.data_ptr(), k.data_ptr(), v.data_ptr(), a.ldp, qnw.data_ptr(),
                        knw.data_ptr(), inv_freq.data_ptr<float>(), pos.data_ptr<int>(),
                        q_out.data_ptr(), kc.data_ptr(), vc.data_ptr(), a.n, a.Hq, a.Hkv,
                        a.max_len, a.rd, (float)eps, stream_of(qg)),
           "qe_attn_prep");
}

// Chunked prefill: q [T, Hq*256] contiguous (normed + roped), kc/vc [Hkv, max_len, 256] holding
// the chunk's K/V (bf16, or E4M3FN codes with kv8), qg rows [T, >= Hq*512] (gate source), out
// rows [T, Hq*256].
struct PrefillArgs {
  int T, Hq, Hkv, max_len;
  long ldp, ldo;
};

PrefillArgs parse_prefill(const torch::Tensor& q, const torch::Tensor& kc, const torch::Tensor& vc,
                          const torch::Tensor& pos, const torch::Tensor& qg,
                          const torch::Tensor& out, bool dev, bool kv8 = false) {
  auto Qr = rows(q, BF, "q", dev), QG = rows(qg, BF, "qg", dev), O = rows(out, BF, "out", dev);
  if (kv8) {
    chk_kv8(kc, "kc8", dev);
    chk_kv8(vc, "vc8", dev);
  } else {
    chk(kc, BF, "kc", dev);
    chk(vc, BF, "vc", dev);
  }
  chk_pos(pos, dev);
  chk16(q, Qr.ld, "q");
  chk16(qg, QG.ld, "qg");
  chk16(out, O.ld, "out");
  chk16(kc, HD, "kc");
  chk16(vc, HD, "vc");
  TORCH_CHECK(kc.dim() == 3 && kc.size(2) == HD && vc.sizes() == kc.sizes(),
              "kc/vc must be [Hkv, max_len, 256] with equal sizes");
  const int T = Qr.n, Hq = Qr.w / HD, Hkv = kc.size(0), max_len = kc.size(1);
  TORCH_CHECK(Hq >= 1 && Qr.ld == Qr.w && QG.n == T && O.n == T && Hq % Hkv == 0,
              "q rows must be contiguous, rows must agree and Hq % Hkv == 0");
  TORCH_CHECK(Qr.w == (long)Hq * HD, "q width must be Hq*256");
  TORCH_CHECK(O.w == (long)Hq * HD && QG.w >= (long)Hq * 2 * HD, "out width Hq*256; qg width Hq*512");
  return {T, Hq, Hkv, max_len, QG.ld, O.ld};
}

void attn_prefill(torch::Tensor q, torch::Tensor kc, torch::Tensor vc, torch::Tensor pos,
                  torch::Tensor qg, torch::Tensor out) {
  const auto a = parse_prefill(q, kc, vc, pos, qg, out, true);
  const c10::DeviceGuard guard(q.device());
  raise_on(qe_attn_prefill(q.data_ptr(), kc.data_ptr(), vc.data_ptr(), pos.data_ptr<int>(),
                           qg.data_ptr(), a.ldp, out.data_ptr(), a.ldo, a.T, a.Hq, a.Hkv,
                           a.max_len, 1.0f / 16.0f, stream_of(q)),
           "qe_attn_prefill");
}

// q: [n, Hq*256] contiguous; part_o: fp32 [>=n, Hq, NS, 256]; part_ml: [>=n, Hq, NS, 2];
// out: [n, Hq*256] gated by sigmoid of the gate half of the qg rows.
void attn_decode(torch::Tensor q, torch::Tensor kc, torch::Tensor vc, torch::Tensor pos,
                 torch::Tensor qg, torch::Tensor part_o, torch::Tensor part_ml, torch::Tensor out) {
  const auto a = parse_decode(q, kc, vc, pos, qg, part_o, part_ml, out, true);
  const c10::DeviceGuard guard(q.device());
  raise_on(qe_attn_decode(q.data_ptr(), kc.data_ptr(), vc.data_ptr(), pos.data_ptr<int>(),
                          qg.data_ptr(), a.ldp, part_o.data_ptr<float>(),
                          part_ml.data_ptr<float>(), out.data_ptr(), a.ldo, a.n, a.Hq, a.Hkv,
                          a.max_len, a.NS, 1.0f / 16.0f /* 256^-0.5 */, stream_of(q)),
           "qe_attn_decode");
}

// attn_prep then attn_decode (q_out is the decode's q) in two launches: the split-KV kernel
// computes its q rows and writes the new cache rows itself. Bit-identical to the two calls.
void attn_prep_decode(torch::Tensor qg, torch::Tensor k, torch::Tensor v, torch::Tensor qnw,
                      torch::Tensor knw, torch::Tensor inv_freq, torch::Tensor pos,
                      torch::Tensor q_out, torch::Tensor kc, torch::Tensor vc, double eps,
                      torch::Tensor part_o, torch::Tensor part_ml, torch::Tensor out) {
  const auto a = parse_prep(qg, k, v, qnw, knw, inv_freq, pos, q_out, kc, vc, true);
  const auto d = parse_decode(q_out, kc, vc, pos, qg, part_o, part_ml, out, true);
  const c10::DeviceGuard guard(qg.device());
  raise_on(qe_attn_prep_decode(qg.data_ptr(), k.data_ptr(), v.data_ptr(), a.ldp, qnw.data_ptr(),
                               knw.data_ptr(), inv_freq.data_ptr<float>(), pos.data_ptr<int>(),
                               q_out.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                               part_o.data_ptr<float>(), part_ml.data_ptr<float>(),
                               out.data_ptr(), d.ldo, a.n, a.Hq, a.Hkv, a.max_len, a.rd, d.NS,
                               1.0f / 16.0f, (float)eps, stream_of(qg)),
           "qe_attn_prep_decode");
}

// The two halves of attn_decode (same arguments): split-KV partials, then the gated combine.
void attn_decode_partials(torch::Tensor q, torch::Tensor kc, torch::Tensor vc, torch::Tensor pos,
                          torch::Tensor qg, torch::Tensor part_o, torch::Tensor part_ml,
                          torch::Tensor out) {
  const auto a = parse_decode(q, kc, vc, pos, qg, part_o, part_ml, out, true);
  const c10::DeviceGuard guard(q.device());
  raise_on(qe_attn_decode_partials(q.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                                   pos.data_ptr<int>(), part_o.data_ptr<float>(),
                                   part_ml.data_ptr<float>(), a.n, a.Hq, a.Hkv, a.max_len, a.NS,
                                   1.0f / 16.0f, stream_of(q)),
           "qe_attn_decode_partials");
}

void attn_decode_combine(torch::Tensor q, torch::Tensor kc, torch::Tensor vc, torch::Tensor pos,
                         torch::Tensor qg, torch::Tensor part_o, torch::Tensor part_ml,
                         torch::Tensor out) {
  const auto a = parse_decode(q, kc, vc, pos, qg, part_o, part_ml, out, true);
  const c10::DeviceGuard guard(q.device());
  raise_on(qe_attn_decode_combine(part_o.data_ptr<float>(), part_ml.data_ptr<float>(),
                                  pos.data_ptr<int>(), qg.data_ptr(), a.ldp, out.data_ptr(),
                                  a.ldo, a.n, a.Hq, a.max_len, a.NS, stream_of(q)),
           "qe_attn_decode_combine");
}

std::vector<int64_t> check_attn_prep(torch::Tensor qg, torch::Tensor k, torch::Tensor v,
                                     torch::Tensor qnw, torch::Tensor knw, torch::Tensor inv_freq,
                                     torch::Tensor pos, torch::Tensor q_out, torch::Tensor kc,
                                     torch::Tensor vc) {
  const auto a = parse_prep(qg, k, v, qnw, knw, inv_freq, pos, q_out, kc, vc, false);
  return {a.n, a.Hq, a.Hkv, a.max_len, a.rd, a.ldp};
}

std::vector<int64_t> check_attn_prep_decode(torch::Tensor qg, torch::Tensor k, torch::Tensor v,
                                            torch::Tensor qnw, torch::Tensor knw,
                                            torch::Tensor inv_freq, torch::Tensor pos,
                                            torch::Tensor q_out, torch::Tensor kc, torch::Tensor vc,
                                            torch::Tensor part_o, torch::Tensor part_ml,
                                            torch::Tensor out) {
  const auto a = parse_prep(qg, k, v, qnw, knw, inv_freq, pos, q_out, kc, vc, false);
  const auto d = parse_decode(q_out, kc, vc, pos, qg, part_o, part_ml, out, false);
  return {a.n, a.Hq, a.Hkv, a.max_len, a.rd, a.ldp, d.NS, d.ldo};
}

std::vector<int64_t> check_attn_decode(torch::Tensor q, torch::Tensor kc, torch::Tensor vc,
                                       torch::Tensor pos, torch::Tensor qg, torch::Tensor part_o,
                                       torch::Tensor part_ml, torch::Tensor out) {
  const auto a = parse_decode(q, kc, vc, pos, qg, part_o, part_ml, out, false);
  return {a.n, a.Hq, a.Hkv, a.max_len, a.NS, a.ldp, a.ldo};
}

// ---- fp8 KV cache (no reference counterpart: the reference cache is bf16, engine.py:419) ------
// attn_prep / attn_decode over a cache of E4M3FN codes with per-cache scales: a stored code c
// means c * scale; prep stores round-to-nearest-even(x / scale), saturated at +-448.
void kv_scales(double k_scale, double v_scale) {
  // as fp32, the kernels' type: normal and finite, so that 1/scale is finite too
  const auto ok = [](double s) {
    const float f = (float)s;
    return f >= std::numeric_limits<float>::min() && f <= std::numeric_limits<float>::max();
  };
  TORCH_CHECK(ok(k_scale) && ok(v_scale),
              "k_scale and v_scale must be positive, finite and not subnormal as fp32");
}

void attn_prep_fp8(torch::Tensor qg, torch::Tensor k, torch::Tensor v, torch::Tensor qnw,
                   torch::Tensor knw, torch::Tensor inv_freq, torch::Tensor pos, torch::Tensor q_out,
                   torch::Tensor kc8, torch::Tensor vc8, double eps, double k_scale,
                   double v_scale) {
  // no reference counterpart: any row count, so it also fills the fp8 cache for prefill chunks
  const auto a = parse_prep(qg, k, v, qnw, knw, inv_freq, pos, q_out, kc8, vc8, true, 65535, true);
  kv_scales(k_scale, v_scale);
  const c10::DeviceGuard guard(qg.device());
  raise_on(qe_attn_prep_fp8(qg.data_ptr(), k.data_ptr(), v.data_ptr(), a.ldp, qnw.data_ptr(),
                            knw.data_ptr(), inv_freq.data_ptr<float>(), pos.data_ptr<int>(),
                            q_out.data_ptr(), kc8.data_ptr(), vc8.data_ptr(), a.n, a.Hq, a.Hkv,
                            a.max_len, a.rd, (float)eps, (float)k_scale, (float)v_scale,
                            stream_of(qg)),
           "qe_attn_prep_fp8");
}

// attn_prefill over the fp8 cache (kc8/vc8 [Hkv, max_len, 256] E4M3FN codes).
void attn_prefill_fp8(torch::Tensor q, torch::Tensor kc8, torch::Tensor vc8, torch::Tensor pos,
                      torch::Tensor qg, torch::Tensor out, double k_scale, double v_scale) {
  kv_scales(k_scale, v_scale);
  const auto a = parse_prefill(q, kc8, vc8, pos, qg, out, true, true);
  const c10::DeviceGuard guard(q.device());
  raise_on(qe_attn_prefill_fp8(q.data_ptr(), kc8.data_ptr(), vc8.data_ptr(), pos.data_ptr<int>(),
                               qg.data_ptr(), a.ldp, out.data_ptr(), a.ldo, a.T, a.Hq, a.Hkv,
                               a.max_len, 1.0f / 16.0f, (float)k_scale, (float)v_scale,
                               stream_of(q)),
           "qe_attn_prefill_fp8");
}

void attn_decode_fp8(torch::Tensor q, torch::Tensor kc8, torch::Tensor vc8, torch::Tensor pos,
                     torch::Tensor qg, torch::Tensor part_o, torch::Tensor part_ml,
                     torch::Tensor out, double k_scale, double v_scale) {
  const auto a = parse_decode(q, kc8, vc8, pos, qg, part_o, part_ml, out, true, true);
  kv_scales(k_scale, v_scale);
  const c10::DeviceGuard guard(q.device());
  raise_on(qe_attn_decode_fp8(q.data_ptr(), kc8.data_ptr(), vc8.data_ptr(), pos.data_ptr<int>(),
                              qg.data_ptr(), a.ldp, part_o.data_ptr<float>(),
                              part_ml.data_ptr<float>(), out.data_ptr(), a.ldo, a.n, a.Hq, a.Hkv,
                              a.max_len, a.NS, 1.0f / 16.0f, (float)k_scale, (float)v_scale,
                              stream_of(q)),
           "qe_attn_decode_fp8");
}

void attn_decode_fp8_partials(torch::Tensor q, torch::Tensor kc8, torch::Tensor vc8,
                              torch::Tensor pos, torch::Tensor qg, torch::Tensor part_o,
                              torch::Tensor part_ml, torch::Tensor out, double k_scale,
                              double v_scale) {
  const auto a = parse_decode(q, kc8, vc8, pos, qg, part_o, part_ml, out, true, true);
  kv_scales(k_scale, v_scale);
  const c10::DeviceGuard guard(q.device());
  raise_on(qe_attn_decode_fp8_partials(q.data_ptr(), kc8.data_ptr(), vc8.data_ptr(),
                                       pos.data_ptr<int>(), part_o.data_ptr<float>(),
                                       part_ml.data_ptr<float>(), a.n, a.Hq, a.Hkv, a.max_len, a.NS,
                                       1.0f / 16.0f, (float)k_scale, stream_of(q)),
           "qe_attn_decode_fp8_partials");
}

// out[n, N] = x[n, K] @ W[N, K]^T for n = 1..8 rows: the reference's gemv_bf16 contract
// (csrc/bindings.cpp:57-66): W contiguous bf16 [N, K], x and out row views, K % 8 == 0,
// 16-byte aligned W and x rows.
struct GemvArgs {
  Rows X, O;
  long N, K;
};
GemvArgs parse_gemv(const torch::Tensor& W, const torch::Tensor& x, const torch::Tensor& out,
                    bool dev) {
  chk(W, BF, "W", dev);
  const auto X = rows(x, BF, "x", dev), O = rows(out, BF, "out", dev);
  TORCH_CHECK(W.dim() == 2 && X.w == W.size(1) && O.w == W.size(0) && X.n == O.n,
              "gemv_bf16: W [N, K], x [n, K], out [n, N]");
  TORCH_CHECK(X.n >= 1 && X.n <= 8, "1..8 rows");
  TORCH_CHECK(W.size(1) % 8 == 0, "K must be a multiple of 8");
  chk16(W, W.size(1), "W");
  chk16(x, X.ld, "x");
  return {X, O, W.size(0), W.size(1)};
}

void gemv_bf16(torch::Tensor W, torch::Tensor x, torch::Tensor out) {
  const auto a = parse_gemv(W, x, out, true);
  TORCH_CHECK(x.device() == W.device() && out.device() == W.device(),
              "W, x and out must be on one device");
  const c10::DeviceGuard guard(W.device());
  raise_on(qe_gemv_bf16(W.data_ptr(), x.data_ptr(), out.data_ptr(), a.X.n, (int)a.N, (int)a.K,
                        a.X.ld, a.O.ld, stream_of(W)),
           "qe_gemv_bf16");
}

std::vector<int64_t> check_gemv_bf16(torch::Tensor W, torch::Tensor x, torch::Tensor out) {
  const auto a = parse_gemv(W, x, out, false);
  return {a.X.n, a.N, a.K, a.X.ld, a.O.ld};
}

// ---- the rest of a decode step (reference csrc/bindings.cpp:33-55,68-136,186-188) ----------
// Each parse_* validates like the reference; dev = false skips the device requirement so the
// _check_* twins can run the contract on a machine without a GPU.

struct EmbedArgs {
  Rows O;
  long V;
};
EmbedArgs parse_embed(const torch::Tensor& table, const torch::Tensor& tok,
                      const torch::Tensor& out, bool dev) {
  chk(table, BF, "table", dev);
  TORCH_CHECK((!dev || tok.is_cuda()) && tok.scalar_type() == I32, "tok must be int32 on the GPU");
  const auto O = rows(out, BF, "out", dev);
  TORCH_CHECK(table.dim() == 2 && O.w == table.size(1) && tok.numel() >= O.n,
              "embed: table [V, H], out [n, H], tok >= n ids");
  return {O, table.size(0)};
}
void embed(torch::Tensor table, torch::Tensor tok, torch::Tensor out) {
  const auto a = parse_embed(table, tok, out, true);
  const c10::DeviceGuard guard(out.device());
  raise_on(qe_embed(table.data_ptr(), tok.data_ptr<int>(), out.data_ptr(), a.O.n, (int)a.O.w,
                    (int)a.V, a.O.ld, stream_of(out)),
           "qe_embed");
}

struct NormArgs {
  Rows X, O;
  long ldd;
  const void* d;
};
NormArgs parse_rmsnorm1p(const torch::Tensor& x, const c10::optional<torch::Tensor>& delta,
                         const torch::Tensor& w, const torch::Tensor& out, bool dev) {
  chk(w, BF, "w", dev);
  const auto X = rows(x, BF, "x", dev), O = rows(out, BF, "out", dev);
  TORCH_CHECK(X.w == w.numel() && O.w == X.w && O.n == X.n, "rmsnorm1p: x [n, H], w [H], out [n, H]");
  long ldd = 0;
  const void* d = nullptr;
  if (delta.has_value()) {
    const auto D = rows(*delta, BF, "delta", dev);
    TORCH_CHECK(D.n == X.n && D.w == X.w, "delta must match x");
    ldd = D.ld;
    d = delta->data_ptr();
  }
  return {X, O, ldd, d};
}
void rmsnorm1p(torch::Tensor x, c10::optional<torch::Tensor> delta, torch::Tensor w,
               torch::Tensor out, double eps) {
  const auto a = parse_rmsnorm1p(x, delta, w, out, true);
  const c10::DeviceGuard guard(x.device());
  raise_on(qe_rmsnorm1p(x.data_ptr(), a.d, w.data_ptr(), out.data_ptr(), a.X.n, (int)a.X.w, a.X.ld,
                        a.ldd, a.O.ld, (float)eps, stream_of(x)),
           "qe_rmsnorm1p");
}

void swiglu(torch::Tensor gu, torch::Tensor out) {
  const auto G = rows(gu, BF, "gu", true), O = rows(out, BF, "out", true);
  TORCH_CHECK(G.w == 2 * O.w && G.n == O.n, "swiglu: gu [n, 2I], out [n, I]");
  const c10::DeviceGuard guard(gu.device());
  raise_on(qe_swiglu(gu.data_ptr(), out.data_ptr(), O.n, (int)O.w, G.ld, O.ld, stream_of(gu)),
           "qe_swiglu");
}

struct ArgmaxArgs {
  Rows X;
  int nb;
  const int* idmap;
};
ArgmaxArgs parse_argmax(const torch::Tensor& x, const torch::Tensor& ws_v,
                        const torch::Tensor& ws_i, const torch::Tensor& out,
                        const c10::optional<torch::Tensor>& idmap, bool dev) {
  const auto X = rows(x, BF, "x", dev);
  chk(ws_v, F32, "ws_v", dev);
  chk(ws_i, I32, "ws_i", dev);
  chk(out, I32, "out", dev);
  const int nb = (int)(ws_v.numel() / X.n);
  TORCH_CHECK(ws_v.numel() == ws_i.numel() && nb >= 1 && out.numel() >= X.n,
              "argmax: ws_v/ws_i of rows*nb entries, out >= rows");
  const int* mp = nullptr;
  if (idmap.has_value()) {
    chk(*idmap, I32, "idmap", dev);
    TORCH_CHECK(idmap->numel() == X.w, "idmap must have one id per column of x");
    mp = idmap->data_ptr<int>();
  }
  return {X, nb, mp};
}
void argmax(torch::Tensor x, torch::Tensor ws_v, torch::Tensor ws_i, torch::Tensor out,
            c10::optional<torch::Tensor> idmap) {
  const auto a = parse_argmax(x, ws_v, ws_i, out, idmap, true);
  const c10::DeviceGuard guard(x.device());
  raise_on(qe_argmax(x.data_ptr(), a.X.n, (int)a.X.w, a.X.ld, ws_v.data_ptr<float>(),
                     ws_i.data_ptr<int>(), a.nb, out.data_ptr<int>(), a.idmap, stream_of(x)),
           "qe_argmax");
}

void parse_accept(const torch::Tensor& in_tok, const torch::Tensor& am, int64_t n,
                  const torch::Tensor& ctl, const torch::Tensor& next_tok,
                  const torch::Tensor& log, bool dev) {
  for (auto* t : {&in_tok, &am, &ctl, &next_tok, &log}) chk(*t, I32, "int buffer", dev);
  TORCH_CHECK(n >= 1 && n <= 8, "accept: 1..8 rows");
  TORCH_CHECK(in_tok.numel() > n && am.numel() >= n && next_tok.numel() >= n && ctl.numel() >= 24,
              "accept: in_tok > n, am and next_tok >= n, ctl >= 24 entries");
}
void accept(torch::Tensor in_tok, torch::Tensor am, int64_t n, torch::Tensor ctl,
            torch::Tensor next_tok, torch::Tensor log) {
  parse_accept(in_tok, am, n, ctl, next_tok, log, true);
  const c10::DeviceGuard guard(ctl.device());
  raise_on(qe_accept(in_tok.data_ptr<int>(), am.data_ptr<int>(), (int)n, ctl.data_ptr<int>(),
                     next_tok.data_ptr<int>(), log.data_ptr<int>(), (int)log.numel(),
                     stream_of(ctl)),
           "qe_accept");
}

void parse_commit(const torch::Tensor& ctl, const torch::Tensor& in_tok, const torch::Tensor& am,
                  const torch::Tensor& drafts, int64_t k, bool dev) {
  for (auto* t : {&ctl, &in_tok, &am, &drafts}) chk(*t, I32, "int buffer", dev);
  TORCH_CHECK(k >= 0 && in_tok.numel() > k && drafts.numel() >= k && ctl.numel() >= 4,
              "commit: in_tok > k, drafts >= k entries");
}
void commit(torch::Tensor ctl, torch::Tensor in_tok, torch::Tensor am, torch::Tensor drafts,
            int64_t k) {
  parse_commit(ctl, in_tok, am, drafts, k, true);
  const c10::DeviceGuard guard(ctl.device());
  raise_on(qe_commit(ctl.data_ptr<int>(), in_tok.data_ptr<int>(), am.data_ptr<int>(),
                     drafts.data_ptr<int>(), (int)k, stream_of(ctl)),
           "qe_commit");
}

struct SelectArgs {
  const void* sp;
  void* dp;
  long lds;
  int H;
};
SelectArgs parse_mtp_select(const torch::Tensor& ctl, const torch::Tensor& mpos,
                            const c10::optional<torch::Tensor>& src,
                            const c10::optional<torch::Tensor>& dst,
                            const c10::optional<torch::Tensor>& mtp_am,
                            const c10::optional<torch::Tensor>& draft0, bool dev) {
  chk(ctl, I32, "ctl", dev);
  chk(mpos, I32, "mpos", dev);
  SelectArgs a{nullptr, nullptr, 0, 0};
  if (src.has_value()) {
    TORCH_CHECK(dst.has_value(), "mtp_select: src needs dst");
    const auto S = rows(*src, BF, "src", dev);
    chk(*dst, BF, "dst", dev);
    TORCH_CHECK(dst->numel() == S.w, "dst must hold one row of src");
    a = {src->data_ptr(), dst->data_ptr(), S.ld, (int)S.w};
  }
  if (draft0.has_value()) {
    TORCH_CHECK(mtp_am.has_value(), "mtp_select: draft0 needs mtp_am");
    chk(*draft0, I32, "draft0", dev);
    chk(*mtp_am, I32, "mtp_am", dev);
  }
  return a;
}
void mtp_select(torch::Tensor ctl, torch::Tensor mpos, int64_t off,
                c10::optional<torch::Tensor> src, c10::optional<torch::Tensor> dst,
                c10::optional<torch::Tensor> mtp_am, c10::optional<torch::Tensor> draft0) {
  const auto a = parse_mtp_select(ctl, mpos, src, dst, mtp_am, draft0, true);
  const c10::DeviceGuard guard(ctl.device());
  raise_on(qe_mtp_select(ctl.data_ptr<int>(), mpos.data_ptr<int>(), (int)off, a.sp, a.lds, a.dp,
                         a.H, mtp_am.has_value() ? mtp_am->data_ptr<int>() : nullptr,
                         draft0.has_value() ? draft0->data_ptr<int>() : nullptr, stream_of(ctl)),
           "qe_mtp_select");
}

// ---- Gated DeltaNet step (reference csrc/bindings.cpp:118-145) -------------------------------
// qkv / z / b / a are row views of one projection buffer sharing a row stride; S is
// [Hv, 128, 128] fp32; the staging buffers hold 8 rows. `q` picks the reference's CUDA block
// shape and is accepted for call compatibility only.
struct GdnArgs {
  int n, Hv;
  long ldp, ldo;
};
GdnArgs parse_gdn(const torch::Tensor& qkv, const torch::Tensor& z, const torch::Tensor& b,
                  const torch::Tensor& a, const torch::Tensor& ring, const torch::Tensor& conv_w,
                  const torch::Tensor& A_log, const torch::Tensor& dt_bias,
                  const torch::Tensor& norm_w, const torch::Tensor& S, const torch::Tensor& st_k,
                  const torch::Tensor& st_v, const torch::Tensor& st_g, const torch::Tensor& ctl,
                  const torch::Tensor& out, int64_t Hk, bool dev) {
  const auto Q = rows(qkv, BF, "qkv", dev), Z = rows(z, BF, "z", dev), B = rows(b, BF, "b", dev),
             A = rows(a, BF, "a", dev), O = rows(out, BF, "out", dev);
  TORCH_CHECK(Q.ld == Z.ld && Q.ld == B.ld && Q.ld == A.ld, "qkv/z/b/a must share a row stride");
  chk(ring, BF, "ring", dev);
  chk(conv_w, BF, "conv_w", dev);
  chk(A_log, BF, "A_log", dev);
  chk(dt_bias, BF, "dt_bias", dev);
  chk(norm_w, BF, "norm_w", dev);
  chk(S, F32, "S", dev);
  chk(st_k, F32, "st_k", dev);
  chk(st_v, F32, "st_v", dev);
  chk(st_g, F32, "st_g", dev);
  chk(ctl, I32, "ctl", dev);
  const int n = Q.n;
  TORCH_CHECK(n >= 1 && n <= 8 && Z.n == n && B.n == n && A.n == n && O.n == n,
              "gdn_step_n: 1..8 rows in every row argument");
  TORCH_CHECK(S.dim() == 3 && S.size(1) == 128 && S.size(2) == 128, "dk = dv = 128 only");
  const long Hv = S.size(0);
  TORCH_CHECK(Hk >= 1 && Hv % Hk == 0, "Hv must be a multiple of Hk");
  const long C = 2 * Hk * 128 + Hv * 128;
  TORCH_CHECK(Q.w == C && ring.numel() == 16 * C && conv_w.numel() == 4 * C,
              "qkv width, ring [16, C] and conv_w [C, 4] must match C = 2*Hk*128 + Hv*128");
  TORCH_CHECK(Z.w == Hv * 128 && O.w == Hv * 128 && B.w == Hv && A.w == Hv,
              "z and out are Hv*128 wide, b and a Hv wide");
  TORCH_CHECK(A_log.numel() == Hv && dt_bias.numel() == Hv && norm_w.numel() == 128,
              "A_log, dt_bias [Hv], norm_w [128]");
  TORCH_CHECK(st_k.numel() == 8L * Hv * 128 && st_v.numel() == 8L * Hv * 128 &&
                  st_g.numel() == 8L * Hv * 2,
              "st_k, st_v [8, Hv, 128], st_g [8, Hv, 2]");
  TORCH_CHECK(ctl.numel() >= 2, "ctl holds pos and pending");
  return {n, (int)Hv, Q.ld, O.ld};
}

void gdn_step_n(torch::Tensor qkv, torch::Tensor z, torch::Tensor b, torch::Tensor a,
                torch::Tensor ring, torch::Tensor conv_w, torch::Tensor A_log,
                torch::Tensor dt_bias, torch::Tensor norm_w, torch::Tensor S, torch::Tensor st_k,
                torch::Tensor st_v, torch::Tensor st_g, torch::Tensor ctl, torch::Tensor out,
                int64_t Hk, double eps, int64_t q) {
  (void)q;
  const auto g = parse_gdn(qkv, z, b, a, ring, conv_w, A_log, dt_bias, norm_w, S, st_k, st_v,
                           st_g, ctl, out, Hk, true);
  const c10::DeviceGuard guard(S.device());
  raise_on(qe_gdn_step_n(qkv.data_ptr(), z.data_ptr(), b.data_ptr(), a.data_ptr(), g.ldp,
                         ring.data_ptr(), conv_w.data_ptr(), A_log.data_ptr(), dt_bias.data_ptr(),
                         norm_w.data_ptr(), S.data_ptr<float>(), st_k.data_ptr<float>(),
                         st_v.data_ptr<float>(), st_g.data_ptr<float>(), ctl.data_ptr<int>(),
                         out.data_ptr(), g.ldo, g.n, (int)Hk, g.Hv, (float)eps, stream_of(S)),
           "qe_gdn_step_n");
}

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.doc() = "MI355X (gfx950) gated-attention decode ops with qengine._C's signatures";
  m.def("attn_prep", &attn_prep);
  m.def("attn_decode", &attn_decode);
  m.def("attn_decode_partials", &attn_decode_partials,
        "split-KV partials of attn_decode (same arguments)");
  m.def("attn_decode_combine", &attn_decode_combine,
        "log-sum-exp combine + sigmoid gate of attn_decode (same arguments)");
  m.def("attn_prep_decode", &attn_prep_decode,
        "attn_prep then attn_decode in two launches (qg, k, v, qnw, knw, inv_freq, pos, q_out, kc, "
        "vc, eps, part_o, part_ml, out)");
  m.def("attn_prep_chunk", &attn_prep_chunk, "attn_prep without the 8-row limit (prefill chunks)");
  m.def("attn_prefill", &attn_prefill,
        "chunked-prefill gated attention over the KV cache (q, kc, vc, pos, qg, out)");
  m.def("split_size", [](int max_len, int NS) { return qe_attn_split_size(max_len, NS); },
        "cache positions per split-KV slice for (max_len, NS)");
  m.def("version", []() { return std::string(qe_attn_version()); });
  m.def("set_pdl_trigger", [](bool on) { qe_set_pdl_trigger(on); },
        "no-op on gfx950 (kept for import compatibility)");
  m.def("set_pdl_launch", [](bool on) { qe_set_pdl_launch(on); },
        "no-op on gfx950 (kept for import compatibility)");
  m.def("_check_attn_prep", &check_attn_prep, "validate attn_prep arguments without launching");
  m.def("_check_attn_prep_decode", &check_attn_prep_decode,
        "validate attn_prep_decode arguments without launching");
  m.def("_check_attn_decode", &check_attn_decode,
        "validate attn_decode arguments without launching");
  m.def("_check_attn_prefill",
        [](torch::Tensor q, torch::Tensor kc, torch::Tensor vc, torch::Tensor pos, torch::Tensor qg,
           torch::Tensor out, bool kv8) {
          const auto a = parse_prefill(q, kc, vc, pos, qg, out, false, kv8);
          return std::vector<int64_t>{a.T, a.Hq, a.Hkv, a.max_len, a.ldp, a.ldo};
        },
        "validate attn_prefill (kv8: attn_prefill_fp8) arguments without launching");
  m.def("_check_kv_scales", [](double k, double v) { kv_scales(k, v); },
        "validate the fp8 cache scales of the *_fp8 ops");
  m.def("gemv_bf16", &gemv_bf16, "out[n, N] = x[n, K] @ W[N, K]^T, n = 1..8 (W, x, out)");
  m.def("attn_prep_fp8", &attn_prep_fp8,
        "attn_prep writing the fp8 KV cache (qg, k, v, qnw, knw, inv_freq, pos, q_out, kc8, vc8, "
        "eps, k_scale, v_scale)");
  m.def("attn_prefill_fp8", &attn_prefill_fp8,
        "attn_prefill over the fp8 cache (q, kc8, vc8, pos, qg, out, k_scale, v_scale)");
  m.def("attn_decode_fp8", &attn_decode_fp8,
        "attn_decode over the fp8 KV cache (q, kc8, vc8, pos, qg, part_o, part_ml, out, k_scale, "
        "v_scale)");
  m.def("attn_decode_fp8_partials", &attn_decode_fp8_partials,
        "split-KV partials of attn_decode_fp8 (same arguments)");
  m.def("_check_attn_decode_fp8", [](torch::Tensor q, torch::Tensor kc8, torch::Tensor vc8,
                                     torch::Tensor pos, torch::Tensor qg, torch::Tensor po,
                                     torch::Tensor pml, torch::Tensor out) {
    const auto a = parse_decode(q, kc8, vc8, pos, qg, po, pml, out, false, true);
    return std::vector<int64_t>{a.n, a.Hq, a.Hkv, a.max_len, a.NS};
  });
  m.def("embed", &embed, "out[r] = table[tok[r]] (zeros for ids outside the table)");
  m.def("rmsnorm1p", &rmsnorm1p, py::arg("x"), py::arg("delta"), py::arg("w"), py::arg("out"),
        py::arg("eps"));
  m.def("swiglu", &swiglu, "out = bf16(bf16(silu(gate)) * up) per row of gu = [gate | up]");
  m.def("argmax", &argmax, py::arg("x"), py::arg("ws_v"), py::arg("ws_i"), py::arg("out"),
        py::arg("idmap") = py::none());
  m.def("accept", &accept);
  m.def("commit", &commit);
  m.def("mtp_select", &mtp_select, py::arg("ctl"), py::arg("mpos"), py::arg("off"),
        py::arg("src") = py::none(), py::arg("dst") = py::none(), py::arg("mtp_am") = py::none(),
        py::arg("draft0") = py::none());
  m.def("l2_persist_limit", [](int64_t b) { raise_on(qe_l2_persist_limit((size_t)b), "qe_l2_persist_limit"); },
        "no-op on gfx950 (no persisting-L2 control; kept for import compatibility)");
  m.def("stream_window",
        [](int64_t base, int64_t bytes, double hit) {
          raise_on(qe_stream_access_window((uintptr_t)base, (size_t)bytes, (float)hit, nullptr),
                   "qe_stream_access_window");
        },
        "no-op on gfx950 (no access-policy window; kept for import compatibility)");
  m.def("_check_embed", [](torch::Tensor t, torch::Tensor k, torch::Tensor o) {
    const auto a = parse_embed(t, k, o, false);
    return std::vector<int64_t>{a.O.n, a.O.w, a.V, a.O.ld};
  });
  m.def("_check_rmsnorm1p", [](torch::Tensor x, c10::optional<torch::Tensor> d, torch::Tensor w,
                               torch::Tensor o) {
    const auto a = parse_rmsnorm1p(x, d, w, o, false);
    return std::vector<int64_t>{a.X.n, a.X.w, a.X.ld, a.ldd, a.O.ld};
  });
  m.def("_check_argmax", [](torch::Tensor x, torch::Tensor v, torch::Tensor i, torch::Tensor o,
                            c10::optional<torch::Tensor> idmap) {
    const auto a = parse_argmax(x, v, i, o, idmap, false);
    return std::vector<int64_t>{a.X.n, a.X.w, a.X.ld, a.nb};
  }, py::arg("x"), py::arg("ws_v"), py::arg("ws_i"), py::arg("out"), py::arg("idmap") = py::none());
  m.def("_check_accept", [](torch::Tensor t, torch::Tensor am, int64_t n, torch::Tensor c,
                            torch::Tensor nt, torch::Tensor lg) {
    parse_accept(t, am, n, c, nt, lg, false);
  });
  m.def("_check_commit", [](torch::Tensor c, torch::Tensor t, torch::Tensor am, torch::Tensor d,
                            int64_t k) { parse_commit(c, t, am, d, k, false); });
  m.def("_check_gemv_bf16", &check_gemv_bf16, "validate gemv_bf16 arguments without launching");
  m.def("gdn_step_n", &gdn_step_n, py::arg("qkv"), py::arg("z"), py::arg("b"), py::arg("a"),
        py::arg("ring"), py::arg("conv_w"), py::arg("A_log"), py::arg("dt_bias"),
        py::arg("norm_w"), py::arg("S"), py::arg("st_k"), py::arg("st_v"), py::arg("st_g"),
        py::arg("ctl"), py::arg("out"), py::arg("Hk"), py::arg("eps"), py::arg("q") = 2,
        "Gated DeltaNet step for n = 1..8 rows with lazy rollback (q: accepted, no effect)");
  m.def("_check_gdn_step_n",
        [](torch::Tensor qkv, torch::Tensor z, torch::Tensor b, torch::Tensor a, torch::Tensor ring,
           torch::Tensor conv_w, torch::Tensor A_log, torch::Tensor dt_bias, torch::Tensor norm_w,
           torch::Tensor S, torch::Tensor st_k, torch::Tensor st_v, torch::Tensor st_g,
           torch::Tensor ctl, torch::Tensor out, int64_t Hk) {
          const auto g = parse_gdn(qkv, z, b, a, ring, conv_w, A_log, dt_bias, norm_w, S, st_k,
                                   st_v, st_g, ctl, out, Hk, false);
          return std::vector<int64_t>{g.n, g.Hv, g.ldp, g.ldo};
        },
        py::arg("qkv"), py::arg("z"), py::arg("b"), py::arg("a"), py::arg("ring"),
        py::arg("conv_w"), py::arg("A_log"), py::arg("dt_bias"), py::arg("norm_w"), py::arg("S"),
        py::arg("st_k"), py::arg("st_v"), py::arg("st_g"), py::arg("ctl"), py::arg("out"),
        py::arg("Hk"), "validate gdn_step_n arguments without launching");
  m.def("set_gdn_phases", [](bool) {},
        "no-op: the reference's phase-parallel A/B switch (one code path here)");
  m.def("set_gdn_early", [](bool) {},
        "no-op: the reference's overlap-with-producer A/B switch (no dependent launch on HIP)");
}

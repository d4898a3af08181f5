// Torch extension `deltanet_chunk_hip`: the drop-in for the reference's
// pybind modules deltanet_chunk_cuda / deltanet_chunk_cuda_tco
// (kernels/torch_binding.cpp:113-131, kernels/torch_binding_tco.cpp).
//
// Same op names, positional order (q, k, v, g, beta, s0) and checks
// (kernels/torch_binding.cpp:28-30,94-101); errors surface as RuntimeError
// through TORCH_CHECK.  Every op allocates its outputs and workspace through
// the caching allocator on the current stream and calls the C ABI of
// libgdn_hip.so (include/gdn_hip.h) with raw pointers; no torch types cross
// that boundary.  New relative to the reference: a trailing keyword
// `cu_seqlens` (varlen prefill), `recurrent_step` (decode),
// `gated_rmsnorm`, `chunk_prefill_norm` (prefill followed by the gated
// RMSNorm, optionally fused into the scan's output stage),
// `chunk_prefill_fused` (the TensorRT adapter's whole GDN step on raw inputs)
// and the causal conv1d ops `causal_conv1d_fwd` / `causal_conv1d_update` that
// produce q/k/v upstream of the recurrence.
#include <torch/extension.h>

// ROCm torch reports HIP devices as DeviceType::CUDA; the *MasqueradingAsCUDA
// guard and stream accessors are the ones that accept those devices.
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>

#include <algorithm>
#include <optional>
#include <vector>

#include "gdn_hip.h"
#include "gdn_hip_diag.h"

namespace {

constexpr int kChunk = 64;

hipStream_t current_stream() { return c10::hip::getCurrentHIPStreamMasqueradingAsCUDA().stream(); }

void check_hip(hipError_t err, const char* what) {
    TORCH_CHECK(err == hipSuccess, what, " failed: ", hipGetErrorString(err));
}

std::vector<at::Tensor> chunk_prefill_impl(const at::Tensor& q, const at::Tensor& k,
                                           const at::Tensor& v, const at::Tensor& g,
                                           const at::Tensor& beta,
                                           const std::optional<at::Tensor>& s0,
                                           const std::optional<at::Tensor>& cu_seqlens,
                                           bool debug, bool qk_l2norm = false,
                                           bool checked = false, int64_t spin = -1) {
    TORCH_CHECK(q.is_cuda() && k.is_cuda() && v.is_cuda() && g.is_cuda() && beta.is_cuda(),
                "all inputs must be CUDA tensors");
    TORCH_CHECK(q.scalar_type() == at::kBFloat16 && k.scalar_type() == at::kBFloat16 &&
                    v.scalar_type() == at::kBFloat16,
                "q/k/v must be bf16");
    TORCH_CHECK(g.scalar_type() == at::kFloat && beta.scalar_type() == at::kFloat,
                "g/beta must be fp32");
    TORCH_CHECK(q.dim() == 4 && k.dim() == 4 && v.dim() == 4 && g.dim() == 3 && beta.dim() == 3,
                "bad ranks");
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(q.device());

    auto qc = q.contiguous();
    auto kc = k.contiguous();
    auto vc = v.contiguous();
    auto gc = g.contiguous();
    auto bc = beta.contiguous();
    const int64_t B = qc.size(0), T = qc.size(1), HQK = qc.size(2), DK = qc.size(3);
    const int64_t HV = vc.size(2), DV = vc.size(3);
    TORCH_CHECK(kc.sizes() == qc.sizes(), "q/k shape mismatch");
    TORCH_CHECK(vc.size(0) == B && vc.size(1) == T && gc.size(0) == B && gc.size(1) == T &&
                    bc.size(0) == B && bc.size(1) == T,
                "batch/time mismatch");
    TORCH_CHECK(kc.size(2) == HQK && gc.size(2) == HV && bc.size(2) == HV, "head-count mismatch");
    TORCH_CHECK(HV % HQK == 0, "HV must be a multiple of HQK");
    TORCH_CHECK(DK == 128 && DV == 128, "only DK = DV = 128 is supported");

    int64_t N = B;
    at::Tensor cu32;
    if (cu_seqlens.has_value()) {
        TORCH_CHECK(cu_seqlens->is_cuda() && cu_seqlens->dim() == 1 && cu_seqlens->numel() >= 2,
                    "cu_seqlens must be a 1-D CUDA tensor [N+1]");
        TORCH_CHECK(cu_seqlens->scalar_type() == at::kInt || cu_seqlens->scalar_type() == at::kLong,
                    "cu_seqlens must be int32 or int64");
        TORCH_CHECK(B == 1, "cu_seqlens requires packed inputs with batch size 1");
        cu32 = cu_seqlens->to(at::kInt).contiguous();
        N = cu32.numel() - 1;
    }

    auto o = at::empty_like(vc);
    auto sf = at::empty({N, HV, DK, DV}, vc.options().dtype(at::kFloat));
    const float* s0p = nullptr;
    at::Tensor s0c;
    if (s0.has_value()) {
        TORCH_CHECK(s0->is_cuda(), "s0 must be a CUDA tensor");
        s0c = s0->to(at::kFloat).contiguous();
        TORCH_CHECK(s0c.dim() == 4 && s0c.size(0) == N && s0c.size(1) == HV && s0c.size(2) == DK &&
                        s0c.size(3) == DV,
                    "s0 must be [N, HV, DK, DV]");
        s0p = s0c.data_ptr<float>();
    }

    // the debug tail only when the views are asked for
    const size_t ws_bytes =
        cu_seqlens.has_value()
            ? (debug ? deltanet_prefill_varlen_workspace_size
                     : deltanet_prefill_varlen_live_workspace_size)((int)T, (int)N, (int)HV,
                                                                    (int)DK, (int)DV, kChunk)
            : (debug ? deltanet_prefill_workspace_size : deltanet_prefill_live_workspace_size)(
                  (int)B, (int)T, (int)HV, (int)DK, (int)DV, kChunk);
    TORCH_CHECK(ws_bytes > 0, "unsupported prefill configuration");
    auto ws = at::empty({(int64_t)ws_bytes}, vc.options().dtype(at::kByte));

    hipError_t err;
    if (spin >= 0) {
        TORCH_CHECK(!qk_l2norm && !cu_seqlens.has_value() && !debug,
                    "the spin-limit test entry takes the plain fixed-length form");
        err = deltanet_chunk_prefill_spin(qc.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                                          gc.data_ptr<float>(), bc.data_ptr<float>(), o.data_ptr(),
                                          s0p, sf.data_ptr<float>(), (int)B, (int)T, (int)HV,
                                          (int)HQK, ws.data_ptr(), ws_bytes, current_stream(),
                                          (unsigned)spin);
    } else if (qk_l2norm) {
        err = deltanet_chunk_prefill_l2norm(
            qc.data_ptr(), kc.data_ptr(), vc.data_ptr(), gc.data_ptr<float>(), bc.data_ptr<float>(),
            o.data_ptr(), s0p, sf.data_ptr<float>(),
            cu_seqlens.has_value() ? cu32.data_ptr<int32_t>() : nullptr, (int)N, (int)B, (int)T,
            (int)HV, (int)HQK, ws.data_ptr(), ws_bytes, current_stream());
    } else if (cu_seqlens.has_value()) {
        err = deltanet_chunk_prefill_varlen(
            qc.data_ptr(), kc.data_ptr(), vc.data_ptr(), gc.data_ptr<float>(), bc.data_ptr<float>(),
            o.data_ptr(), s0p, sf.data_ptr<float>(), cu32.data_ptr<int32_t>(), (int)N, (int)T,
            (int)HV, (int)HQK, (int)DK, (int)DV, kChunk, ws.data_ptr(), ws_bytes,
            current_stream(), debug ? 1 : 0);
    } else {
        err = deltanet_chunk_prefill(qc.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                                     gc.data_ptr<float>(), bc.data_ptr<float>(), o.data_ptr(), s0p,
                                     sf.data_ptr<float>(), (int)B, (int)T, (int)HV, (int)HQK,
                                     (int)DK, (int)DV, kChunk, ws.data_ptr(), ws_bytes,
                                     current_stream(), debug ? 1 : 0);
    }
    check_hip(err, "deltanet_chunk_prefill");
    if (checked || spin >= 0) {
        const hipError_t st = deltanet_prefill_status(ws.data_ptr(), ws_bytes, current_stream());
        if (spin >= 0) {
            // test entry: the status is returned, not raised
            auto flag = at::full({1}, st == hipSuccess ? 0 : 1, vc.options().dtype(at::kInt));
            return {o, sf, flag};
        }
        check_hip(st, "deltanet_chunk_prefill (status word)");
    }

    std::vector<at::Tensor> out{o, sf};
    if (debug) {
        // debug tail, the last six regions of the workspace, each 256-byte
        // aligned (gdn_prefill.hip WsLayout): per chunk-head fp32 T, A,
        // T after the diagonal blocks, M ([64][64] each), cumsum(g) [64] and
        // the state at the chunk's start [128][128]
        const int64_t nc = cu_seqlens.has_value() ? (T + (int64_t)(kChunk - 1) * N) / kChunk
                                                  : B * ((T + kChunk - 1) / kChunk);
        const int64_t nch = nc * HV;
        auto al = [](int64_t b) { return (b + 255) & ~int64_t(255); };
        const int64_t sq = al(nch * kChunk * kChunk * 4), sc = al(nch * kChunk * 4),
                      ss = al(nch * DK * DV * 4);
        const int64_t off = (int64_t)ws_bytes - (4 * sq + sc + ss);
        auto wsf = [&](int64_t byte_off, int64_t count) {
            return ws.narrow(0, byte_off, count * 4).view(at::kFloat);
        };
        out.push_back(wsf(off, nch * kChunk * kChunk).view({nc, HV, kChunk, kChunk}));            // T
        out.push_back(wsf(off + sq, nch * kChunk * kChunk).view({nc, HV, kChunk, kChunk}));       // A
        out.push_back(wsf(off + 4 * sq, nch * kChunk).view({nc, HV, kChunk}));                   // cumsum g
        out.push_back(wsf(off + 2 * sq, nch * kChunk * kChunk).view({nc, HV, kChunk, kChunk}));   // T post-leaf
        out.push_back(wsf(off + 3 * sq, nch * kChunk * kChunk).view({nc, HV, kChunk, kChunk}));   // M
        out.push_back(wsf(off + 4 * sq + sc, nch * DK * DV).view({nc, HV, DK, DV}));              // S_c
    }
    return out;
}

}  // namespace

std::vector<at::Tensor> chunk_prefill(at::Tensor q, at::Tensor k, at::Tensor v, at::Tensor g,
                                      at::Tensor beta, std::optional<at::Tensor> s0,
                                      std::optional<at::Tensor> cu_seqlens, bool qk_l2norm,
                                      bool checked) {
    return chunk_prefill_impl(q, k, v, g, beta, s0, cu_seqlens, /*debug=*/false, qk_l2norm,
                              checked);
}

// Test entry: the plain prefill with the scan's bounded waits limited to
// `spin` polls; returns [o, final_state, status] with status 1 when a wait
// gave up (o and final_state are then incomplete).
std::vector<at::Tensor> chunk_prefill_spin_limit(at::Tensor q, at::Tensor k, at::Tensor v,
                                                 at::Tensor g, at::Tensor beta,
                                                 std::optional<at::Tensor> s0, int64_t spin) {
    TORCH_CHECK(spin >= 0, "spin must be >= 0");
    return chunk_prefill_impl(q, k, v, g, beta, s0, std::nullopt, /*debug=*/false, false, false,
                              spin);
}

std::vector<at::Tensor> chunk_prefill_debug(at::Tensor q, at::Tensor k, at::Tensor v,
                                            at::Tensor g, at::Tensor beta,
                                            std::optional<at::Tensor> s0,
                                            std::optional<at::Tensor> cu_seqlens) {
    return chunk_prefill_impl(q, k, v, g, beta, s0, cu_seqlens, /*debug=*/true);
}

// Prefill followed by the gated RMSNorm: returns [y, final_state], y =
// gated_rmsnorm(o, z, weight, eps) for the o that chunk_prefill would return
// (bf16 o, z and weight).  fused=True runs the RMSNorm inside the scan
// (deltanet_chunk_prefill_norm_fused; the same bits).
std::vector<at::Tensor> chunk_prefill_norm(at::Tensor q, at::Tensor k, at::Tensor v, at::Tensor g,
                                           at::Tensor beta, at::Tensor z, at::Tensor weight,
                                           std::optional<at::Tensor> s0, double eps,
                                           bool checked, bool fused) {
    TORCH_CHECK(q.is_cuda() && k.is_cuda() && v.is_cuda() && g.is_cuda() && beta.is_cuda() &&
                    z.is_cuda() && weight.is_cuda(),
                "all inputs must be CUDA tensors");
    TORCH_CHECK(q.scalar_type() == at::kBFloat16 && k.scalar_type() == at::kBFloat16 &&
                    v.scalar_type() == at::kBFloat16 && z.scalar_type() == at::kBFloat16 &&
                    weight.scalar_type() == at::kBFloat16,
                "q/k/v/z/weight must be bf16");
    TORCH_CHECK(g.scalar_type() == at::kFloat && beta.scalar_type() == at::kFloat,
                "g/beta must be fp32");
    TORCH_CHECK(q.dim() == 4 && k.dim() == 4 && v.dim() == 4 && g.dim() == 3 && beta.dim() == 3,
                "bad ranks");
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(q.device());
    auto qc = q.contiguous();
    auto kc = k.contiguous();
    auto vc = v.contiguous();
    auto gc = g.contiguous();
    auto bc = beta.contiguous();
    auto zc = z.contiguous();
    auto wc = weight.contiguous();
    const int64_t B = qc.size(0), T = qc.size(1), HQK = qc.size(2), DK = qc.size(3);
    const int64_t HV = vc.size(2), DV = vc.size(3);
    TORCH_CHECK(kc.sizes() == qc.sizes(), "q/k shape mismatch");
    TORCH_CHECK(vc.size(0) == B && vc.size(1) == T && gc.size(0) == B && gc.size(1) == T &&
                    gc.size(2) == HV && bc.sizes() == gc.sizes(),
                "batch/time/head mismatch");
    TORCH_CHECK(zc.sizes() == vc.sizes(), "z must have v's shape [B, T, HV, 128]");
    TORCH_CHECK(wc.dim() == 1 && wc.size(0) == DV, "weight must be [128]");
    TORCH_CHECK(HV % HQK == 0, "HV must be a multiple of HQK");
    TORCH_CHECK(DK == 128 && DV == 128, "only DK = DV = 128 is supported");
    auto y = at::empty_like(vc);
    auto sf = at::empty({B, HV, DK, DV}, vc.options().dtype(at::kFloat));
    const float* s0p = nullptr;
    at::Tensor s0c;
    if (s0.has_value()) {
        TORCH_CHECK(s0->is_cuda(), "s0 must be a CUDA tensor");
        s0c = s0->to(at::kFloat).contiguous();
        TORCH_CHECK(s0c.dim() == 4 && s0c.size(0) == B && s0c.size(1) == HV &&
                        s0c.size(2) == DK && s0c.size(3) == DV,
                    "s0 must be [B, HV, DK, DV]");
        s0p = s0c.data_ptr<float>();
    }
    const size_t ws_bytes = deltanet_prefill_live_workspace_size((int)B, (int)T, (int)HV, (int)DK,
                                                                 (int)DV, kChunk);
    TORCH_CHECK(ws_bytes > 0, "unsupported prefill configuration");
    auto ws = at::empty({(int64_t)ws_bytes}, vc.options().dtype(at::kByte));
    auto entry = fused ? deltanet_chunk_prefill_norm_fused : deltanet_chunk_prefill_norm;
    check_hip(entry(qc.data_ptr(), kc.data_ptr(), vc.data_ptr(), gc.data_ptr<float>(),
                    bc.data_ptr<float>(), zc.data_ptr(), wc.data_ptr(), (float)eps, y.data_ptr(),
                    s0p, sf.data_ptr<float>(), (int)B, (int)T, (int)HV, (int)HQK, (int)DK,
                    (int)DV, kChunk, ws.data_ptr(), ws_bytes, current_stream()),
              "deltanet_chunk_prefill_norm");
    if (checked)
        check_hip(deltanet_prefill_status(ws.data_ptr(), ws_bytes, current_stream()),
                  "deltanet_chunk_prefill_norm (status word)");
    return {y, sf};
}

at::Tensor recurrent_step(at::Tensor q, at::Tensor k, at::Tensor v, at::Tensor g,
                          at::Tensor beta, at::Tensor state, bool qk_l2norm) {
    TORCH_CHECK(q.is_cuda() && k.is_cuda() && v.is_cuda() && g.is_cuda() && beta.is_cuda() &&
                    state.is_cuda(),
                "all inputs must be CUDA tensors");
    TORCH_CHECK(q.scalar_type() == at::kBFloat16 && k.scalar_type() == at::kBFloat16 &&
                    v.scalar_type() == at::kBFloat16,
                "q/k/v must be bf16");
    TORCH_CHECK(g.scalar_type() == at::kFloat && beta.scalar_type() == at::kFloat &&
                    state.scalar_type() == at::kFloat,
                "g/beta/state must be fp32");
    TORCH_CHECK(q.dim() == 4 && k.dim() == 4 && v.dim() == 4 && g.dim() == 3 && beta.dim() == 3 &&
                    state.dim() == 4,
                "bad ranks");
    TORCH_CHECK(state.is_contiguous(), "state is updated in place and must be contiguous");
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(q.device());
    auto qc = q.contiguous();
    auto kc = k.contiguous();
    auto vc = v.contiguous();
    auto gc = g.contiguous();
    auto bc = beta.contiguous();
    const int64_t B = qc.size(0), T = qc.size(1), HQK = qc.size(2), DK = qc.size(3);
    const int64_t HV = vc.size(2), DV = vc.size(3);
    TORCH_CHECK(kc.sizes() == qc.sizes(), "q/k shape mismatch");
    TORCH_CHECK(vc.size(0) == B && vc.size(1) == T && gc.size(0) == B && gc.size(1) == T &&
                    gc.size(2) == HV && bc.sizes() == gc.sizes(),
                "batch/time/head mismatch");
    TORCH_CHECK(HV % HQK == 0, "HV must be a multiple of HQK");
    TORCH_CHECK(state.size(0) == B && state.size(1) == HV && state.size(2) == DK &&
                    state.size(3) == DV,
                "state must be [B, HV, DK, DV]");
    auto o = at::empty_like(vc);
    auto step = qk_l2norm ? deltanet_recurrent_step_l2norm : deltanet_recurrent_step;
    check_hip(step(qc.data_ptr(), kc.data_ptr(), vc.data_ptr(), gc.data_ptr<float>(),
                   bc.data_ptr<float>(), o.data_ptr(), state.data_ptr<float>(), (int)B, (int)T,
                   (int)HV, (int)HQK, (int)DK, (int)DV, current_stream()),
              "deltanet_recurrent_step");
    return o;
}

at::Tensor gated_rmsnorm(at::Tensor x, at::Tensor z, at::Tensor weight, double eps) {
    TORCH_CHECK(x.is_cuda() && z.is_cuda() && weight.is_cuda(), "all inputs must be CUDA tensors");
    TORCH_CHECK(x.scalar_type() == at::kBFloat16 || x.scalar_type() == at::kHalf,
                "x must be bf16 or fp16");
    TORCH_CHECK(z.scalar_type() == x.scalar_type(), "z must have the dtype of x");
    TORCH_CHECK(weight.scalar_type() == x.scalar_type() || weight.scalar_type() == at::kFloat,
                "weight must have the dtype of x or be fp32");
    TORCH_CHECK(x.sizes() == z.sizes(), "x/z shape mismatch");
    TORCH_CHECK(x.dim() >= 1 && weight.dim() == 1 && weight.size(0) == x.size(-1),
                "weight must be [x.size(-1)]");
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
    auto xc = x.contiguous();
    auto zc = z.contiguous();
    auto wc = weight.contiguous();
    auto y = at::empty_like(xc);
    const int dv = (int)xc.size(-1);
    const int64_t rows = dv > 0 ? xc.numel() / dv : 0;
    const int io = x.scalar_type() == at::kBFloat16 ? GDN_DTYPE_BF16 : GDN_DTYPE_FP16;
    const int wd = weight.scalar_type() == at::kFloat ? GDN_DTYPE_FP32 : io;
    check_hip(gdn_gated_rmsnorm_forward(xc.data_ptr(), zc.data_ptr(), wc.data_ptr(), y.data_ptr(),
                                        rows, dv, (float)eps, io, wd, current_stream()),
              "gdn_gated_rmsnorm_forward");
    return y;
}

// The reference TensorRT adapter's whole GDN step on raw inputs
// (gdnChunkPrefillSm87.cu:189-316) as one op: q, k [B, T, HQK, 128] raw;
// v [B, T, HV, 128]; a, b [B, T, HV]; A_log [HV] (fp32); dt_bias [HV];
// state [B, HV, 128, 128] fp32, initial on entry, final on return.  q, k,
// v, a, b, dt_bias share one dtype (fp16 or bf16), which o gets too.
at::Tensor chunk_prefill_fused(at::Tensor q, at::Tensor k, at::Tensor v, at::Tensor a,
                               at::Tensor b, at::Tensor A_log, at::Tensor dt_bias,
                               at::Tensor state) {
    for (const at::Tensor* t : {&q, &k, &v, &a, &b, &A_log, &dt_bias, &state})
        TORCH_CHECK(t->is_cuda(), "all inputs must be CUDA tensors");
    const auto dt = q.scalar_type();
    TORCH_CHECK(dt == at::kHalf || dt == at::kBFloat16, "q must be fp16 or bf16");
    TORCH_CHECK(k.scalar_type() == dt && v.scalar_type() == dt && a.scalar_type() == dt &&
                    b.scalar_type() == dt && dt_bias.scalar_type() == dt,
                "q, k, v, a, b and dt_bias must share one dtype");
    TORCH_CHECK(A_log.scalar_type() == at::kFloat, "A_log must be fp32");
    TORCH_CHECK(state.scalar_type() == at::kFloat && state.is_contiguous(),
                "state must be a contiguous fp32 tensor (updated in place)");
    TORCH_CHECK(q.dim() == 4 && k.sizes() == q.sizes() && v.dim() == 4 && a.dim() == 3 &&
                    b.sizes() == a.sizes(),
                "bad ranks or shapes");
    const int64_t B = q.size(0), T = q.size(1), HQK = q.size(2), HV = v.size(2);
    TORCH_CHECK(q.size(3) == 128 && v.size(3) == 128, "only head dims of 128 are supported");
    TORCH_CHECK(v.size(0) == B && v.size(1) == T && a.size(0) == B && a.size(1) == T &&
                    a.size(2) == HV,
                "batch/time/head mismatch");
    TORCH_CHECK(HV % HQK == 0, "HV must be a multiple of HQK");
    TORCH_CHECK(A_log.numel() == HV && dt_bias.numel() == HV, "A_log and dt_bias must be [HV]");
    TORCH_CHECK(state.dim() == 4 && state.size(0) == B && state.size(1) == HV &&
                    state.size(2) == 128 && state.size(3) == 128,
                "state must be [B, HV, 128, 128]");
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(q.device());
    auto qc = q.contiguous(), kc = k.contiguous(), vc = v.contiguous();
    auto ac = a.contiguous(), bc = b.contiguous();
    auto Ac = A_log.contiguous(), dc = dt_bias.contiguous();
    auto o = at::empty_like(vc);
    const size_t ws_bytes =
        deltanet_prefill_live_workspace_size((int)B, (int)T, (int)HV, 128, 128, kChunk);
    TORCH_CHECK(ws_bytes > 0 || T == 0, "unsupported prefill configuration");
    auto ws = at::empty({(int64_t)std::max<size_t>(ws_bytes, 256)}, vc.options().dtype(at::kByte));
    check_hip(deltanet_chunk_prefill_fused(
                  qc.data_ptr(), kc.data_ptr(), vc.data_ptr(), ac.data_ptr(), bc.data_ptr(),
                  Ac.data_ptr<float>(), dc.data_ptr(), o.data_ptr(), state.data_ptr<float>(),
                  (int)B, (int)T, (int)HV, (int)HQK,
                  dt == at::kHalf ? GDN_DTYPE_FP16 : GDN_DTYPE_BF16, ws.data_ptr(),
                  (size_t)ws.numel(),
                  current_stream()),
              "deltanet_chunk_prefill_fused");
    return o;
}

int conv_io_dtype(const at::Tensor& x) {
    TORCH_CHECK(x.scalar_type() == at::kBFloat16 || x.scalar_type() == at::kHalf,
                "x must be bf16 or fp16");
    return x.scalar_type() == at::kBFloat16 ? GDN_DTYPE_BF16 : GDN_DTYPE_FP16;
}

int conv_w_dtype(const at::Tensor& x, const at::Tensor& w, const std::optional<at::Tensor>& bias) {
    TORCH_CHECK(w.scalar_type() == x.scalar_type() || w.scalar_type() == at::kFloat,
                "weight must have the dtype of x or be fp32");
    TORCH_CHECK(!bias || bias->scalar_type() == w.scalar_type(),
                "bias must have the dtype of weight");
    return w.scalar_type() == at::kFloat ? GDN_DTYPE_FP32 : conv_io_dtype(x);
}

// x: [B, D, T] (a transposed view of a channel-contiguous [B, T, D] buffer is
// used as is; anything else is first copied into that layout), weight
// [D, K], bias [D] or None.  Returns y: [B, D, T], a view of a contiguous
// [B, T, D] buffer (so y.transpose(1, 2) is contiguous).
at::Tensor causal_conv1d_fwd(const at::Tensor& x, const at::Tensor& weight,
                             const std::optional<at::Tensor>& bias, bool silu) {
    TORCH_CHECK(x.is_cuda() && weight.is_cuda() && (!bias || bias->is_cuda()),
                "all inputs must be CUDA tensors");
    TORCH_CHECK(x.dim() == 3, "x must be [B, D, T]");
    const int64_t B = x.size(0), D = x.size(1), T = x.size(2);
    TORCH_CHECK(weight.dim() == 2 && weight.size(0) == D, "weight must be [D, K]");
    TORCH_CHECK(!bias || (bias->dim() == 1 && bias->size(0) == D), "bias must be [D]");
    TORCH_CHECK(D % 8 == 0, "the channel count must be a multiple of 8");
    const int io = conv_io_dtype(x), wd = conv_w_dtype(x, weight, bias);
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
    auto xt = x.transpose(1, 2);   // [B, T, D]
    const bool direct = xt.stride(2) == 1 && (B <= 1 || xt.stride(0) % 8 == 0) &&
                        (T <= 1 || xt.stride(1) % 8 == 0) &&
                        reinterpret_cast<uintptr_t>(xt.data_ptr()) % 16 == 0;
    if (!direct) xt = xt.contiguous();
    auto wc = weight.contiguous();
    std::optional<at::Tensor> bc;
    if (bias) bc = bias->contiguous();
    auto yt = at::empty({B, T, D}, x.options());
    check_hip(gdn_causal_conv1d_fwd(xt.data_ptr(), wc.data_ptr(), bc ? bc->data_ptr() : nullptr,
                                    yt.data_ptr(), (int)B, (int)T, (int)D, (int)wc.size(1),
                                    B <= 1 ? 0 : xt.stride(0), T <= 1 ? 0 : xt.stride(1),
                                    yt.stride(0), yt.stride(1), io, wd, silu ? 1 : 0,
                                    current_stream()),
              "gdn_causal_conv1d_fwd");
    return yt.transpose(1, 2);
}

// x: [B, D, T] (any strides), conv_state: [B, D, L] with unit token stride,
// updated in place; weight [D, K]; bias [D] or None.  Returns y [B, D, T]
// laid out like causal_conv1d_fwd's.
at::Tensor causal_conv1d_update(const at::Tensor& x, at::Tensor conv_state,
                                const at::Tensor& weight, const std::optional<at::Tensor>& bias,
                                bool silu) {
    TORCH_CHECK(x.is_cuda() && conv_state.is_cuda() && weight.is_cuda() &&
                    (!bias || bias->is_cuda()),
                "all inputs must be CUDA tensors");
    TORCH_CHECK(x.dim() == 3, "x must be [B, D, T]");
    const int64_t B = x.size(0), D = x.size(1), T = x.size(2);
    TORCH_CHECK(conv_state.dim() == 3 && conv_state.size(0) == B && conv_state.size(1) == D,
                "conv_state must be [B, D, L]");
    TORCH_CHECK(conv_state.scalar_type() == x.scalar_type(), "conv_state must have the dtype of x");
    TORCH_CHECK(conv_state.stride(2) == 1 || conv_state.size(2) == 1,
                "conv_state must have unit stride along its last dimension");
    TORCH_CHECK(weight.dim() == 2 && weight.size(0) == D, "weight must be [D, K]");
    TORCH_CHECK(!bias || (bias->dim() == 1 && bias->size(0) == D), "bias must be [D]");
    const int io = conv_io_dtype(x), wd = conv_w_dtype(x, weight, bias);
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
    auto wc = weight.contiguous();
    std::optional<at::Tensor> bc;
    if (bias) bc = bias->contiguous();
    auto y = at::empty({B, T, D}, x.options()).transpose(1, 2);
    check_hip(gdn_causal_conv1d_update(x.data_ptr(), conv_state.data_ptr(), wc.data_ptr(),
                                       bc ? bc->data_ptr() : nullptr, y.data_ptr(), (int)B, (int)T,
                                       (int)D, (int)wc.size(1), (int)conv_state.size(2),
                                       x.stride(0), x.stride(2), x.stride(1), conv_state.stride(0),
                                       conv_state.stride(1), y.stride(0), y.stride(2), y.stride(1),
                                       io, wd, silu ? 1 : 0, current_stream()),
              "gdn_causal_conv1d_update");
    return y;
}

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    using namespace pybind11::literals;
    m.def("chunk_prefill", &chunk_prefill,
          "chunked gated delta rule prefill (gfx950 HIP); returns [o, final_state]; qk_l2norm: "
          "q and k rows are raw and L2-normalised in the kernel",
          "q"_a, "k"_a, "v"_a, "g"_a, "beta"_a, "s0"_a = std::nullopt, pybind11::kw_only(),
          "cu_seqlens"_a = std::nullopt, "qk_l2norm"_a = false, "checked"_a = false);
    m.def("chunk_prefill_debug", &chunk_prefill_debug,
          "same, also returns per-chunk-head views: T=(I-A)^-1, A, cumsum(g), T after the "
          "diagonal-block inversion, M, and the state at each chunk's start",
          "q"_a, "k"_a, "v"_a, "g"_a, "beta"_a, "s0"_a = std::nullopt, pybind11::kw_only(),
          "cu_seqlens"_a = std::nullopt);
    m.def("chunk_prefill_norm", &chunk_prefill_norm,
          "prefill followed by the gated RMSNorm; returns [y, final_state], y = "
          "gated_rmsnorm(o, z, weight, eps) for chunk_prefill's o; fused=True runs the norm in "
          "the scan's output stage",
          "q"_a, "k"_a, "v"_a, "g"_a, "beta"_a, "z"_a, "weight"_a, "s0"_a = std::nullopt,
          pybind11::kw_only(), "eps"_a = 1e-6, "checked"_a = false, "fused"_a = false);
    m.def("_chunk_prefill_spin_limit", &chunk_prefill_spin_limit,
          "test entry: prefill with the scan's bounded waits limited to `spin` polls; returns "
          "[o, final_state, status]",
          "q"_a, "k"_a, "v"_a, "g"_a, "beta"_a, "s0"_a, "spin"_a);
    m.def("recurrent_step", &recurrent_step,
          "recurrent gated delta rule (decode), state updated in place; returns o", "q"_a, "k"_a,
          "v"_a, "g"_a, "beta"_a, "state"_a, pybind11::kw_only(), "qk_l2norm"_a = false);
    m.def("chunk_prefill_fused", &chunk_prefill_fused,
          "prefill on raw inputs (q/k L2 norm, gates, dtype conversions fused); state updated "
          "in place; returns o",
          "q"_a, "k"_a, "v"_a, "a"_a, "b"_a, "A_log"_a, "dt_bias"_a, "state"_a);
    m.def("gated_rmsnorm", &gated_rmsnorm, "y = rmsnorm(x) * weight * silu(z)", "x"_a, "z"_a,
          "weight"_a, "eps"_a = 1e-6);
    m.def("causal_conv1d_fwd", &causal_conv1d_fwd,
          "causal depthwise conv1d over x [B, D, T] with optional SiLU; returns y [B, D, T]",
          "x"_a, "weight"_a, "bias"_a = std::nullopt, "silu"_a = false);
    m.def("causal_conv1d_update", &causal_conv1d_update,
          "decode-time causal conv1d; conv_state [B, D, L] updated in place; returns y", "x"_a,
          "conv_state"_a, "weight"_a, "bias"_a = std::nullopt, "silu"_a = false);
}

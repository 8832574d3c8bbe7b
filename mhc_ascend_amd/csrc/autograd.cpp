// Autograd nodes of the fused mHC layers in C++ over the C ABI of
// libmhc_hip (the role of the reference's Python autograd functions,
// src/python/mhc/ops.py:387-564, and of its pybind11 layer entries,
// src/python/bindings.cpp:600-952).  Forward and backward prepare their
// arguments exactly as mhc_ascend_amd/native.py does (same checks, dtypes,
// workspaces and error text) and call the same entry points, so results are
// identical bit for bit; doing it in C++ keeps the interpreter out of the
// forward and the autograd engine's hand-off to a Python backward out of
// every step.
//
// The fused MHCResidualWrapper (layer.py:269-322) has nodes of the same kind.
// These nodes are the package's only orchestration of the fused entries;
// tests/pyref_autograd.py restates them in Python for a bit-for-bit check.
//
// The entry points are not linked: bind() receives their addresses from the
// ctypes handle of the already loaded library, so both paths share one copy
// of it (one error state, one set of per-device caches) whichever build of
// it was loaded.
#include <torch/extension.h>

#include <ATen/hip/HIPContext.h>

#include <algorithm>
#include <map>
#include <string>
#include <vector>

#include "mhc_hip.h"

namespace {

using torch::Tensor;
using torch::autograd::AutogradContext;
using torch::autograd::tensor_list;

#define MHC_AUTOGRAD_ENTRIES(X)               \
    X(mhc_last_error)                         \
    X(mhc_layer_static_saved_size)            \
    X(mhc_layer_static_fwd)                   \
    X(mhc_layer_static_bwd_workspace_size)    \
    X(mhc_layer_static_bwd)                   \
    X(mhc_layer_dynamic_saved_size)           \
    X(mhc_layer_dynamic_fwd_workspace_size)   \
    X(mhc_layer_dynamic_fwd)                  \
    X(mhc_layer_dynamic_bwd_workspace_size)   \
    X(mhc_layer_dynamic_bwd)                  \
    X(mhc_wrapper_dynamic_saved_size)         \
    X(mhc_wrapper_dynamic_fwd_workspace_size_for) \
    X(mhc_wrapper_dynamic_fwd)                \
    X(mhc_wrapper_dynamic_bwd_workspace_size_for) \
    X(mhc_wrapper_dynamic_bwd)                \
    X(mhc_wrapper_static_fwd)                 \
    X(mhc_wrapper_static_bwd_workspace_size)  \
    X(mhc_wrapper_static_bwd)

struct Entries {
#define MHC_DECLARE(name) decltype(&::name) name = nullptr;
    MHC_AUTOGRAD_ENTRIES(MHC_DECLARE)
#undef MHC_DECLARE
};

Entries lib;
bool bound = false;

void bind(const std::map<std::string, int64_t>& addrs) {
    Entries e;
#define MHC_BIND(name)                                                                            \
    {                                                                                             \
        auto it = addrs.find(#name);                                                              \
        TORCH_CHECK(it != addrs.end() && it->second != 0, "mhc autograd: no address for " #name); \
        e.name = reinterpret_cast<decltype(e.name)>(static_cast<intptr_t>(it->second));           \
    }
    MHC_AUTOGRAD_ENTRIES(MHC_BIND)
#undef MHC_BIND
    lib = e;
    bound = true;
}

std::vector<std::string> entry_names() {
    return {
#define MHC_NAME(name) #name,
        MHC_AUTOGRAD_ENTRIES(MHC_NAME)
#undef MHC_NAME
    };
}

void require_bound() { TORCH_CHECK(bound, "mhc autograd: bind() the HIP library's entry points first"); }

int dtype_code(at::ScalarType t) {
    if (t == at::kFloat) return MHC_DTYPE_F32;
    if (t == at::kBFloat16) return MHC_DTYPE_BF16;
    TORCH_CHECK(false, "mhc_ascend_amd: unsupported storage dtype ", t, " (float32 or bfloat16)");
    return -1;
}

void check(int rc, const char* name) {
    TORCH_CHECK(rc == 0, name, " failed (status ", rc, "): ", lib.mhc_last_error());
}

void check_device(const char* fn, std::initializer_list<const Tensor*> ts) {
    c10::optional<c10::Device> dev;
    for (const Tensor* t : ts) {
        TORCH_CHECK(t->is_cuda(), fn, ": tensors must be on a HIP device (got ", t->device(),
                    "); mhc_ascend_amd has no CPU path");
        if (!dev) {
            dev = t->device();
        } else {
            TORCH_CHECK(t->device() == *dev, fn, ": all tensors must be on the same device (", *dev, " vs ",
                        t->device(), ")");
        }
    }
}

bool storage_dtype(at::ScalarType t) { return t == at::kFloat || t == at::kBFloat16; }

Tensor layer_x(const char* fn, const Tensor& x) {
    TORCH_CHECK(x.dim() == 3, fn, ": x must be 3D [B, n, C]");
    return (storage_dtype(x.scalar_type()) ? x : x.to(at::kFloat)).contiguous();
}

Tensor weight(const Tensor& w) { return (storage_dtype(w.scalar_type()) ? w : w.to(at::kFloat)).contiguous(); }

Tensor f32c(const Tensor& t) { return t.to(at::kFloat).contiguous(); }

// alpha as a 1-element fp32 device tensor (a device pointer: no host sync)
Tensor scalar_param(const Tensor& a, c10::Device dev) {
    return a.detach().to(dev, at::kFloat).reshape({1}).contiguous();
}

Tensor workspace(size_t nbytes, const Tensor& like) {
    return at::empty({(int64_t)std::max<size_t>(nbytes, 1)}, like.options().dtype(at::kByte));
}

void* stream() { return at::hip::getCurrentHIPStream().stream(); }

float* fp(const Tensor& t) { return t.data_ptr<float>(); }

// ---- static H: mhc_ascend_amd.ops.MHCLayerStaticFunction (layer.py:142-170) --
struct StaticLayer : public torch::autograd::Function<StaticLayer> {
    static Tensor forward(AutogradContext* ctx, const Tensor& x_in, const Tensor& w_in, const Tensor& hp_in,
                          const Tensor& hq_in, const Tensor& hr_in, int64_t iters, double sk_eps, double rms_eps) {
        const char* fn = "mhc_layer_static_fwd";
        check_device(fn, {&x_in, &w_in, &hp_in, &hq_in, &hr_in});
        const at::DeviceGuard guard(x_in.device());
        const Tensor x = layer_x(fn, x_in);
        const int64_t B = x.size(0), n = x.size(1), C = x.size(2);
        TORCH_CHECK(w_in.numel() == C && hp_in.numel() == n && hq_in.numel() == n && hr_in.numel() == n * n,
                    "mhc_layer_static_fwd: parameter shapes do not match x [B, n, C]");
        const Tensor w = weight(w_in), hp = f32c(hp_in), hq = f32c(hq_in), hr = f32c(hr_in);
        const auto f32 = x.options().dtype(at::kFloat);
        Tensor out = at::empty({B, n, C}, f32);
        Tensor rms = at::empty({B}, f32);
        Tensor saved = at::empty({(int64_t)(lib.mhc_layer_static_saved_size((int32_t)n, (int32_t)C) / 4)}, f32);
        check(lib.mhc_layer_static_fwd(x.data_ptr(), dtype_code(x.scalar_type()), w.data_ptr(),
                                       dtype_code(w.scalar_type()), fp(hp), fp(hq), fp(hr), fp(out), fp(rms),
                                       fp(saved), B, (int32_t)n, (int32_t)C, (int32_t)iters, (float)sk_eps,
                                       (float)rms_eps, stream()),
              fn);
        ctx->save_for_backward({x, w, hp, hq, hr, saved});
        ctx->saved_data["x_dtype"] = (int64_t)x_in.scalar_type();
        ctx->saved_data["hp_shape"] = hp_in.sizes().vec();
        ctx->saved_data["hq_shape"] = hq_in.sizes().vec();
        ctx->saved_data["hr_shape"] = hr_in.sizes().vec();
        ctx->saved_data["cfg"] = std::vector<double>{(double)iters, sk_eps, rms_eps};
        return out;
    }

    static tensor_list backward(AutogradContext* ctx, tensor_list grads) {
        const char* fn = "mhc_layer_static_bwd";
        const auto sv = ctx->get_saved_variables();
        const Tensor &x = sv[0], &w = sv[1], &hp = sv[2], &hq = sv[3], &hr = sv[4], &saved = sv[5];
        check_device(fn, {&grads[0], &x});
        const at::DeviceGuard guard(x.device());
        const auto cfg = ctx->saved_data["cfg"].toDoubleVector();
        const int64_t B = x.size(0), n = x.size(1), C = x.size(2);
        TORCH_CHECK(grads[0].sizes() == x.sizes(), "mhc_layer_static_bwd: grad_out must match x [B, n, C]");
        const Tensor g = f32c(grads[0]);
        const auto f32 = x.options().dtype(at::kFloat);
        Tensor grad_x = at::empty_like(x);
        Tensor gw = at::empty({C}, w.options());
        Tensor ghp = at::empty({n}, f32), ghq = at::empty({n}, f32), ghr = at::empty({n, n}, f32);
        const int xd = dtype_code(x.scalar_type());
        const size_t wsb = lib.mhc_layer_static_bwd_workspace_size(B, (int32_t)n, (int32_t)C, xd);
        Tensor ws = workspace(wsb, x);
        check(lib.mhc_layer_static_bwd(fp(g), x.data_ptr(), xd, dtype_code(w.scalar_type()), fp(hp), fp(hq), fp(hr),
                                       fp(saved), grad_x.data_ptr(), gw.data_ptr(), fp(ghp), fp(ghq), fp(ghr),
                                       ws.data_ptr(), wsb, B, (int32_t)n, (int32_t)C, (int32_t)cfg[0],
                                       (float)cfg[1], (float)cfg[2], stream()),
              fn);
        const auto x_dtype = (at::ScalarType)ctx->saved_data["x_dtype"].toInt();
        return {grad_x.to(x_dtype),
                gw,
                ghp.view(ctx->saved_data["hp_shape"].toIntVector()),
                ghq.view(ctx->saved_data["hq_shape"].toIntVector()),
                ghr.view(ctx->saved_data["hr_shape"].toIntVector()),
                Tensor(),
                Tensor(),
                Tensor()};
    }
};

// ---- dynamic H: mhc_ascend_amd.ops.MHCLayerDynamicFunction (ops.py:387-564) --
std::vector<Tensor> phi_parts(const Tensor& pre, const Tensor& post, const Tensor& res, int64_t n, int64_t nC) {
    std::vector<Tensor> parts = {f32c(pre), f32c(post), f32c(res)};
    const int64_t rows[3] = {n, n, n * n};
    for (int i = 0; i < 3; ++i) {
        TORCH_CHECK(parts[i].numel() == rows[i] * nC, "dynamic layer: projection of ", parts[i].sizes(),
                    " does not match [", rows[i], ", ", nC, "]");
    }
    return parts;
}

struct DynamicLayer : public torch::autograd::Function<DynamicLayer> {
    static Tensor forward(AutogradContext* ctx, const Tensor& x_in, const Tensor& w_in, const Tensor& pp_in,
                          const Tensor& pq_in, const Tensor& pr_in, const Tensor& ap_in, const Tensor& aq_in,
                          const Tensor& ar_in, const Tensor& bp_in, const Tensor& bq_in, const Tensor& br_in,
                          int64_t iters, double sk_eps, double rms_eps) {
        const char* fn = "mhc_layer_dynamic_fwd";
        check_device(fn, {&x_in, &w_in, &pp_in, &pq_in, &pr_in, &bp_in, &bq_in, &br_in});
        const at::DeviceGuard guard(x_in.device());
        const Tensor x = layer_x(fn, x_in);
        const int64_t B = x.size(0), n = x.size(1), C = x.size(2);
        const Tensor w = weight(w_in);
        TORCH_CHECK(w.numel() == C, "mhc_layer_dynamic_fwd: rmsnorm_weight must have C elements");
        const auto ph = phi_parts(pp_in, pq_in, pr_in, n, n * C);
        const Tensor ap = scalar_param(ap_in, x.device()), aq = scalar_param(aq_in, x.device()),
                     ar = scalar_param(ar_in, x.device());
        const Tensor bp = f32c(bp_in), bq = f32c(bq_in), br = f32c(br_in);
        const auto f32 = x.options().dtype(at::kFloat);
        Tensor out = at::empty({B, n, C}, f32);
        Tensor saved = at::empty({(int64_t)(lib.mhc_layer_dynamic_saved_size(B, (int32_t)n, (int32_t)C) / 4)}, f32);
        const size_t wsb = lib.mhc_layer_dynamic_fwd_workspace_size(B, (int32_t)n, (int32_t)C);
        Tensor ws = workspace(wsb, x);
        check(lib.mhc_layer_dynamic_fwd(x.data_ptr(), dtype_code(x.scalar_type()), w.data_ptr(),
                                        dtype_code(w.scalar_type()), fp(ph[0]), fp(ph[1]), fp(ph[2]), fp(ap), fp(aq),
                                        fp(ar), fp(bp), fp(bq), fp(br), fp(out), fp(saved), ws.data_ptr(), wsb, B,
                                        (int32_t)n, (int32_t)C, (int32_t)iters, (float)sk_eps, (float)rms_eps,
                                        stream()),
              fn);
        ctx->save_for_backward({x, w, saved, ph[0], ph[1], ph[2], ap, aq, ar, bp, bq, br});
        ctx->saved_data["x_dtype"] = (int64_t)x_in.scalar_type();
        std::vector<int64_t> shapes;  // rank, then sizes, of each parameter in argument order
        for (const Tensor* t : {&pp_in, &pq_in, &pr_in, &ap_in, &aq_in, &ar_in, &bp_in, &bq_in, &br_in}) {
            shapes.push_back(t->dim());
            for (int64_t s : t->sizes()) shapes.push_back(s);
        }
        ctx->saved_data["shapes"] = shapes;
        ctx->saved_data["cfg"] = std::vector<double>{(double)iters, sk_eps, rms_eps};
        return out;
    }

    static tensor_list backward(AutogradContext* ctx, tensor_list grads) {
        const char* fn = "mhc_layer_dynamic_bwd";
        const auto sv = ctx->get_saved_variables();
        const Tensor &x = sv[0], &w = sv[1], &saved = sv[2];
        check_device(fn, {&grads[0], &x});
        const at::DeviceGuard guard(x.device());
        const auto cfg = ctx->saved_data["cfg"].toDoubleVector();
        const int64_t B = x.size(0), n = x.size(1), C = x.size(2), np = 2 * n + n * n;
        TORCH_CHECK(grads[0].sizes() == x.sizes(), "mhc_layer_dynamic_bwd: grad_output must match x [B, n, C]");
        const Tensor g = f32c(grads[0]);
        const auto f32 = x.options().dtype(at::kFloat);
        Tensor grad_x = at::empty_like(x);
        Tensor gw = at::empty({C}, w.options());
        Tensor gphi = at::empty({np, n * C}, f32);
        Tensor galpha = at::empty({3}, f32);
        Tensor gb = at::empty({np}, f32);
        const int xd = dtype_code(x.scalar_type());
        const size_t wsb = lib.mhc_layer_dynamic_bwd_workspace_size(B, (int32_t)n, (int32_t)C, xd);
        Tensor ws = workspace(wsb, x);
        check(lib.mhc_layer_dynamic_bwd(fp(g), x.data_ptr(), xd, dtype_code(w.scalar_type()), fp(sv[3]), fp(sv[4]),
                                        fp(sv[5]), fp(sv[6]), fp(sv[7]), fp(sv[8]), fp(sv[9]), fp(sv[10]),
                                        fp(sv[11]), fp(saved), grad_x.data_ptr(), gw.data_ptr(), fp(gphi),
                                        fp(galpha), fp(gb), ws.data_ptr(), wsb, B, (int32_t)n, (int32_t)C,
                                        (int32_t)cfg[0], (float)cfg[1], (float)cfg[2], stream()),
              fn);
        const auto flat = ctx->saved_data["shapes"].toIntVector();
        std::vector<std::vector<int64_t>> shp;
        for (size_t i = 0; i < flat.size();) {
            const int64_t r = flat[i++];
            shp.emplace_back(flat.begin() + i, flat.begin() + i + r);
            i += r;
        }
        const auto x_dtype = (at::ScalarType)ctx->saved_data["x_dtype"].toInt();
        return {grad_x.to(x_dtype),
                gw,
                gphi.narrow(0, 0, n).view(shp[0]),
                gphi.narrow(0, n, n).view(shp[1]),
                gphi.narrow(0, 2 * n, n * n).view(shp[2]),
                galpha.narrow(0, 0, 1).view(shp[3]),
                galpha.narrow(0, 1, 1).view(shp[4]),
                galpha.narrow(0, 2, 1).view(shp[5]),
                gb.narrow(0, 0, n).view(shp[6]),
                gb.narrow(0, n, n).view(shp[7]),
                gb.narrow(0, 2 * n, n * n).view(shp[8]),
                Tensor(),
                Tensor(),
                Tensor()};
    }
};

// ---- fused MHCResidualWrapper (layer.py:269-322) ----------------------------
std::vector<int64_t> flat_shapes(std::initializer_list<const Tensor*> ts) {
    std::vector<int64_t> v;  // rank, then sizes, of each tensor in order
    for (const Tensor* t : ts) {
        v.push_back(t->dim());
        for (int64_t d : t->sizes()) v.push_back(d);
    }
    return v;
}

std::vector<std::vector<int64_t>> unflat_shapes(const std::vector<int64_t>& flat) {
    std::vector<std::vector<int64_t>> out;
    for (size_t i = 0; i < flat.size();) {
        const int64_t r = flat[i++];
        out.emplace_back(flat.begin() + i, flat.begin() + i + r);
        i += r;
    }
    return out;
}

// residual / branch [tokens, hidden] as the kernels read them: residual in
// fp32 or bf16 (others become fp32), branch in the residual's dtype.
std::pair<Tensor, Tensor> wrapper_inputs(const char* fn, const Tensor& residual, const Tensor& branch) {
    check_device(fn, {&residual, &branch});
    TORCH_CHECK(residual.sizes() == branch.sizes() && residual.dim() == 2, fn,
                ": residual and branch must both be [tokens, hidden] of one shape");
    Tensor r = (storage_dtype(residual.scalar_type()) ? residual : residual.to(at::kFloat)).contiguous();
    return {r, branch.to(r.scalar_type()).contiguous()};
}

int32_t wrapper_mode(const std::string& mode, int64_t n, const char* fn) {
    TORCH_CHECK_VALUE(mode == "decay" || mode == "zero", "Unknown residual_mode: ", mode);
    // the reference writes stream 1 (layer.py:301), which needs n >= 2
    TORCH_CHECK(n >= 2, fn, ": expansion_rate must be >= 2 (stream 1 holds the branch)");
    return mode == "decay" ? MHC_WRAPPER_DECAY : MHC_WRAPPER_ZERO;
}

struct StaticWrapper : public torch::autograd::Function<StaticWrapper> {
    static Tensor forward(AutogradContext* ctx, const Tensor& res_in, const Tensor& br_in, const Tensor& w_in,
                          const Tensor& hp_in, const Tensor& hq_in, const Tensor& hr_in, int64_t mode, int64_t n,
                          int64_t iters, double sk_eps, double rms_eps) {
        const char* fn = "wrapper_static_fwd";
        auto [r, b] = wrapper_inputs(fn, res_in, br_in);
        check_device(fn, {&r, &w_in, &hp_in, &hq_in, &hr_in});
        const at::DeviceGuard guard(r.device());
        const int64_t T = r.size(0), C = r.size(1);
        const Tensor w = weight(w_in);
        TORCH_CHECK(w.numel() == C && hp_in.numel() == n && hq_in.numel() == n && hr_in.numel() == n * n,
                    "wrapper_static_fwd: parameter shapes do not match n and C");
        const Tensor hp = f32c(hp_in), hq = f32c(hq_in), hr = f32c(hr_in);
        const auto f32 = r.options().dtype(at::kFloat);
        Tensor out = at::empty({T, C}, f32);
        Tensor saved = at::empty({(int64_t)(lib.mhc_layer_static_saved_size((int32_t)n, (int32_t)C) / 4)}, f32);
        check(lib.mhc_wrapper_static_fwd(r.data_ptr(), b.data_ptr(), dtype_code(r.scalar_type()), (int32_t)mode,
                                         w.data_ptr(), dtype_code(w.scalar_type()), fp(hp), fp(hq), fp(hr), fp(out),
                                         fp(saved), T, (int32_t)n, (int32_t)C, (int32_t)iters, (float)sk_eps,
                                         (float)rms_eps, stream()),
              "mhc_wrapper_static_fwd");
        ctx->save_for_backward({r, b, w, hp, hq, hr, saved});
        ctx->saved_data["dtypes"] = std::vector<int64_t>{(int64_t)res_in.scalar_type(), (int64_t)br_in.scalar_type()};
        ctx->saved_data["shapes"] = flat_shapes({&hp_in, &hq_in, &hr_in});
        ctx->saved_data["cfg"] = std::vector<double>{(double)mode, (double)n, (double)iters, sk_eps, rms_eps};
        return out;
    }

    static tensor_list backward(AutogradContext* ctx, tensor_list grads) {
        const char* fn = "wrapper_static_bwd";
        const auto sv = ctx->get_saved_variables();
        const Tensor &r = sv[0], &b = sv[1], &w = sv[2], &saved = sv[6];
        check_device(fn, {&grads[0], &r});
        const at::DeviceGuard guard(r.device());
        const auto cfg = ctx->saved_data["cfg"].toDoubleVector();
        const int64_t T = r.size(0), C = r.size(1), n = (int64_t)cfg[1];
        const int32_t mode = (int32_t)cfg[0];
        TORCH_CHECK(grads[0].sizes() == r.sizes(), "wrapper_static_bwd: grad_out must be [tokens, hidden]");
        const Tensor g = f32c(grads[0]);
        const auto f32 = r.options().dtype(at::kFloat);
        Tensor gr = at::empty_like(r), gb = at::empty_like(b);
        Tensor gw = at::empty({C}, w.options());
        Tensor ghp = at::empty({n}, f32), ghq = at::empty({n}, f32), ghr = at::empty({n, n}, f32);
        const int dt = dtype_code(r.scalar_type());
        const size_t wsb = lib.mhc_wrapper_static_bwd_workspace_size(T, (int32_t)n, (int32_t)C, dt, mode);
        Tensor ws = workspace(wsb, r);
        check(lib.mhc_wrapper_static_bwd(fp(g), r.data_ptr(), b.data_ptr(), dt, mode, dtype_code(w.scalar_type()),
                                         fp(sv[3]), fp(sv[4]), fp(sv[5]), fp(saved), gr.data_ptr(), gb.data_ptr(),
                                         gw.data_ptr(), fp(ghp), fp(ghq), fp(ghr), ws.data_ptr(), wsb, T, (int32_t)n,
                                         (int32_t)C, (int32_t)cfg[2], (float)cfg[3], (float)cfg[4], stream()),
              "mhc_wrapper_static_bwd");
        const auto dts = ctx->saved_data["dtypes"].toIntVector();
        const auto shp = unflat_shapes(ctx->saved_data["shapes"].toIntVector());
        return {gr.to((at::ScalarType)dts[0]), gb.to((at::ScalarType)dts[1]), gw, ghp.view(shp[0]), ghq.view(shp[1]),
                ghr.view(shp[2]), Tensor(), Tensor(), Tensor(), Tensor(), Tensor()};
    }
};

struct DynamicWrapper : public torch::autograd::Function<DynamicWrapper> {
    static Tensor forward(AutogradContext* ctx, const Tensor& res_in, const Tensor& br_in, const Tensor& w_in,
                          const Tensor& pp_in, const Tensor& pq_in, const Tensor& pr_in, const Tensor& ap_in,
                          const Tensor& aq_in, const Tensor& ar_in, const Tensor& bp_in, const Tensor& bq_in,
                          const Tensor& bres_in, int64_t mode, int64_t n, int64_t iters, double sk_eps,
                          double rms_eps) {
        const char* fn = "wrapper_dynamic_fwd";
        auto [r, b] = wrapper_inputs(fn, res_in, br_in);
        check_device(fn, {&r, &w_in, &pp_in, &pq_in, &pr_in, &bp_in, &bq_in, &bres_in});
        const at::DeviceGuard guard(r.device());
        const int64_t T = r.size(0), C = r.size(1);
        const Tensor w = weight(w_in);
        TORCH_CHECK(w.numel() == C, "wrapper_dynamic_fwd: rmsnorm_weight must have C elements");
        const auto ph = phi_parts(pp_in, pq_in, pr_in, n, n * C);
        const Tensor ap = scalar_param(ap_in, r.device()), aq = scalar_param(aq_in, r.device()),
                     ar = scalar_param(ar_in, r.device());
        const Tensor bp = f32c(bp_in), bq = f32c(bq_in), bres = f32c(bres_in);
        const auto f32 = r.options().dtype(at::kFloat);
        Tensor out = at::empty({T, C}, f32);
        Tensor saved =
            at::empty({(int64_t)(lib.mhc_wrapper_dynamic_saved_size(T, (int32_t)n, (int32_t)C) / 4)}, f32);
        const size_t wsb = lib.mhc_wrapper_dynamic_fwd_workspace_size_for(T, (int32_t)n, (int32_t)C,
                                                                          dtype_code(r.scalar_type()));
        Tensor ws = workspace(wsb, r);
        check(lib.mhc_wrapper_dynamic_fwd(r.data_ptr(), b.data_ptr(), dtype_code(r.scalar_type()), (int32_t)mode,
                                          w.data_ptr(), dtype_code(w.scalar_type()), fp(ph[0]), fp(ph[1]), fp(ph[2]),
                                          fp(ap), fp(aq), fp(ar), fp(bp), fp(bq), fp(bres), fp(out), fp(saved),
                                          ws.data_ptr(), wsb, T, (int32_t)n, (int32_t)C, (int32_t)iters,
                                          (float)sk_eps, (float)rms_eps, stream()),
              "mhc_wrapper_dynamic_fwd");
        ctx->save_for_backward({r, b, w, saved, ph[0], ph[1], ph[2], ap, aq, ar, bres});
        ctx->saved_data["dtypes"] = std::vector<int64_t>{(int64_t)res_in.scalar_type(), (int64_t)br_in.scalar_type()};
        ctx->saved_data["shapes"] =
            flat_shapes({&pp_in, &pq_in, &pr_in, &ap_in, &aq_in, &ar_in, &bp_in, &bq_in, &bres_in});
        ctx->saved_data["cfg"] = std::vector<double>{(double)mode, (double)n, (double)iters, sk_eps, rms_eps};
        return out;
    }

    static tensor_list backward(AutogradContext* ctx, tensor_list grads) {
        const char* fn = "wrapper_dynamic_bwd";
        const auto sv = ctx->get_saved_variables();
        const Tensor &r = sv[0], &b = sv[1], &w = sv[2], &saved = sv[3];
        check_device(fn, {&grads[0], &r});
        const at::DeviceGuard guard(r.device());
        const auto cfg = ctx->saved_data["cfg"].toDoubleVector();
        const int64_t T = r.size(0), C = r.size(1), n = (int64_t)cfg[1], np = 2 * n + n * n;
        const int32_t mode = (int32_t)cfg[0];
        TORCH_CHECK(grads[0].sizes() == r.sizes(), "wrapper_dynamic_bwd: grad_out must be [tokens, hidden]");
        const Tensor g = f32c(grads[0]);
        const auto f32 = r.options().dtype(at::kFloat);
        Tensor gr = at::empty_like(r), gb = at::empty_like(b);
        Tensor gw = at::empty({C}, w.options());
        Tensor gphi = at::empty({np, n * C}, f32);
        Tensor galpha = at::empty({3}, f32);
        Tensor gbias = at::empty({np}, f32);
        const int dt = dtype_code(r.scalar_type());
        const size_t wsb = lib.mhc_wrapper_dynamic_bwd_workspace_size_for(T, (int32_t)n, (int32_t)C, dt, mode,
                                                                          (int32_t)cfg[2], (float)cfg[3]);
        Tensor ws = workspace(wsb, r);
        check(lib.mhc_wrapper_dynamic_bwd(fp(g), r.data_ptr(), b.data_ptr(), dt, mode, dtype_code(w.scalar_type()),
                                          fp(sv[4]), fp(sv[5]), fp(sv[6]), fp(sv[7]), fp(sv[8]), fp(sv[9]),
                                          fp(sv[10]), fp(saved), gr.data_ptr(), gb.data_ptr(), gw.data_ptr(),
                                          fp(gphi), fp(galpha), fp(gbias), ws.data_ptr(), wsb, T, (int32_t)n,
                                          (int32_t)C, (int32_t)cfg[2], (float)cfg[3], (float)cfg[4], stream()),
              "mhc_wrapper_dynamic_bwd");
        const auto dts = ctx->saved_data["dtypes"].toIntVector();
        const auto shp = unflat_shapes(ctx->saved_data["shapes"].toIntVector());
        return {gr.to((at::ScalarType)dts[0]),
                gb.to((at::ScalarType)dts[1]),
                gw,
                gphi.narrow(0, 0, n).view(shp[0]),
                gphi.narrow(0, n, n).view(shp[1]),
                gphi.narrow(0, 2 * n, n * n).view(shp[2]),
                galpha.narrow(0, 0, 1).view(shp[3]),
                galpha.narrow(0, 1, 1).view(shp[4]),
                galpha.narrow(0, 2, 1).view(shp[5]),
                gbias.narrow(0, 0, n).view(shp[6]),
                gbias.narrow(0, n, n).view(shp[7]),
                gbias.narrow(0, 2 * n, n * n).view(shp[8]),
                Tensor(),
                Tensor(),
                Tensor(),
                Tensor(),
                Tensor()};
    }
};

Tensor static_layer(const Tensor& x, const Tensor& w, const Tensor& hp, const Tensor& hq, const Tensor& hr,
                    int64_t iters, double sk_eps, double rms_eps) {
    require_bound();
    return StaticLayer::apply(x, w, hp, hq, hr, iters, sk_eps, rms_eps);
}

Tensor dynamic_layer(const Tensor& x, const Tensor& w, const Tensor& pp, const Tensor& pq, const Tensor& pr,
                     const Tensor& ap, const Tensor& aq, const Tensor& ar, const Tensor& bp, const Tensor& bq,
                     const Tensor& br, int64_t iters, double sk_eps, double rms_eps) {
    require_bound();
    return DynamicLayer::apply(x, w, pp, pq, pr, ap, aq, ar, bp, bq, br, iters, sk_eps, rms_eps);
}

Tensor static_wrapper(const Tensor& residual, const Tensor& branch, const Tensor& w, const Tensor& hp,
                      const Tensor& hq, const Tensor& hr, const std::string& mode, int64_t n, int64_t iters,
                      double sk_eps, double rms_eps) {
    require_bound();
    const int32_t m = wrapper_mode(mode, n, "wrapper_static_fwd");
    return StaticWrapper::apply(residual, branch, w, hp, hq, hr, (int64_t)m, n, iters, sk_eps, rms_eps);
}

Tensor dynamic_wrapper(const Tensor& residual, const Tensor& branch, const Tensor& w, const Tensor& pp,
                       const Tensor& pq, const Tensor& pr, const Tensor& ap, const Tensor& aq, const Tensor& ar,
                       const Tensor& bp, const Tensor& bq, const Tensor& bres, const std::string& mode, int64_t n,
                       int64_t iters, double sk_eps, double rms_eps) {
    require_bound();
    const int32_t m = wrapper_mode(mode, n, "wrapper_dynamic_fwd");
    return DynamicWrapper::apply(residual, branch, w, pp, pq, pr, ap, aq, ar, bp, bq, bres, (int64_t)m, n, iters,
                                 sk_eps, rms_eps);
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    m.doc() = "C++ autograd nodes of the fused mHC layers over libmhc_hip's C ABI";
    m.def("entry_names", &entry_names, "C-ABI entry points bind() needs");
    m.def("bind", &bind, "set the C-ABI entry points from {name: address}");
    m.def("static_layer", &static_layer,
          "static-H layer with autograd: (x, weight, H_pre, H_post, H_res, num_iters, sinkhorn_eps, "
          "rmsnorm_eps) -> fp32 [B, n, C]");
    m.def("dynamic_layer", &dynamic_layer,
          "dynamic-H layer with autograd: (x, weight, phi_pre, phi_post, phi_res, alpha_pre, alpha_post, "
          "alpha_res, b_pre, b_post, b_res, num_iters, sinkhorn_eps, rmsnorm_eps) -> fp32 [B, n, C]");
    m.def("static_wrapper", &static_wrapper,
          "fused static-H MHCResidualWrapper with autograd: (residual, branch, weight, H_pre, H_post, H_res, "
          "residual_mode, n, num_iters, sinkhorn_eps, rmsnorm_eps) -> fp32 [tokens, C]");
    m.def("dynamic_wrapper", &dynamic_wrapper,
          "fused dynamic-H MHCResidualWrapper with autograd: (residual, branch, weight, phi_pre, phi_post, phi_res, "
          "alpha_pre, alpha_post, alpha_res, b_pre, b_post, b_res, residual_mode, n, num_iters, sinkhorn_eps, "
          "rmsnorm_eps) -> fp32 [tokens, C]");
}

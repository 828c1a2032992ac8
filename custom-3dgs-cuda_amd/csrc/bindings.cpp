// bindings.cpp — the pybind11 module `custom_rasterizer_cuda`: the reference's
// six-function surface (csrc/bindings.cpp:141-153 of kmurungi/custom-3dgs-cuda)
// with the same positional arguments, tensor layouts, return tuples, checks
// and messages, implemented over the C ABI of libgsraster.so.  Outputs come
// from torch's caching allocator on the inputs' device; every launch goes on
// torch's current HIP stream.
#include <torch/extension.h>

#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>

#include <tuple>
#include <vector>

#include "../../include/gsraster.h"

namespace {

using torch::Tensor;

// The reference's validation macros (csrc/cuda_check.h:23-47).
#define CHECK_CUDA(tensor) TORCH_CHECK((tensor).is_cuda(), #tensor " must be a CUDA tensor")
#define CHECK_CONTIGUOUS(tensor) TORCH_CHECK((tensor).is_contiguous(), #tensor " must be contiguous")
#define CHECK_FP32(tensor) \
    TORCH_CHECK((tensor).scalar_type() == torch::kFloat32, #tensor " must be FP32")
#define CHECK_INT32(tensor) \
    TORCH_CHECK((tensor).scalar_type() == torch::kInt32, #tensor " must be int32")
#define CHECK_INPUT_FP32(tensor) \
    do {                         \
        CHECK_CUDA(tensor);      \
        CHECK_CONTIGUOUS(tensor);\
        CHECK_FP32(tensor);      \
    } while (0)
#define CHECK_INPUT_INT32(tensor) \
    do {                          \
        CHECK_CUDA(tensor);       \
        CHECK_CONTIGUOUS(tensor); \
        CHECK_INT32(tensor);      \
    } while (0)

void check_rc(int rc, const char* what) {
    TORCH_CHECK(rc == GSR_OK, "custom_rasterizer_cuda.", what, ": ", gsr_last_error());
}

void* current_stream() {
    return static_cast<void*>(c10::hip::getCurrentHIPStreamMasqueradingAsCUDA().stream());
}

float* fp(const Tensor& t) { return t.data_ptr<float>(); }
const float* cfp(const Tensor& t) { return t.data_ptr<float>(); }

Tensor workspace(int64_t bytes, const Tensor& like) {
    return torch::empty({std::max<int64_t>(bytes, 1)},
                        torch::TensorOptions().dtype(torch::kUInt8).device(like.device()));
}

void check_numel(const Tensor& t, int64_t want, const char* msg) {
    TORCH_CHECK(t.numel() >= want, msg);
}

// The kernels read quaternions and SH coefficients in 16-byte units; a
// contiguous view that starts mid-allocation is copied to fresh storage.
Tensor aligned16(const Tensor& t) {
    return (reinterpret_cast<uintptr_t>(t.data_ptr()) & 15) ? t.clone() : t;
}

// ---- project (bindings.cpp:12-29 / projection.cu:109-153) ----
std::tuple<Tensor, Tensor, Tensor> project(int total_gaussians, const Tensor mu3d,
                                           const Tensor q3d, const Tensor s3d,
                                           const Tensor camera_rotation,
                                           const Tensor camera_translation, float fx, float fy,
                                           float cx, float cy) {
    CHECK_INPUT_FP32(mu3d);
    CHECK_INPUT_FP32(q3d);
    CHECK_INPUT_FP32(s3d);
    CHECK_INPUT_FP32(camera_rotation);
    CHECK_INPUT_FP32(camera_translation);
    TORCH_CHECK(total_gaussians >= 0, "total_gaussians must be non-negative");
    const int64_t n = total_gaussians;
    check_numel(mu3d, 3 * n, "mu3d must hold N x 3 values");
    check_numel(q3d, 4 * n, "q3d must hold N x 4 values");
    check_numel(s3d, 3 * n, "s3d must hold N x 3 values");
    check_numel(camera_rotation, 9, "camera_rotation must hold 3 x 3 values");
    check_numel(camera_translation, 3, "camera_translation must hold 3 values");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(mu3d.device());
    auto options = torch::TensorOptions().dtype(torch::kFloat32).device(mu3d.device());
    Tensor mean_2d = torch::empty({n, 2}, options);
    Tensor cov_2d = torch::empty({n, 3}, options);
    Tensor depths = torch::empty({n}, options);
    const Tensor q_al = aligned16(q3d);
    check_rc(gsr_project(total_gaussians, cfp(mu3d), cfp(q_al), cfp(s3d), cfp(camera_rotation),
                         cfp(camera_translation), fx, fy, cx, cy, fp(mean_2d), fp(cov_2d),
                         fp(depths), current_stream()),
             "project");
    return {mean_2d, cov_2d, depths};
}

// ---- glue helpers (no counterpart in the reference's module; used by the
// autograd glue in place of its torch ops, rasterize.py:43-53) ----
Tensor screen_radii(const Tensor cov_2d) {
    CHECK_INPUT_FP32(cov_2d);
    TORCH_CHECK(cov_2d.dim() == 2 && cov_2d.size(1) == 3, "cov_2d must have shape (N, 3)");
    const int64_t n = cov_2d.size(0);
    c10::hip::HIPGuardMasqueradingAsCUDA guard(cov_2d.device());
    Tensor radii = torch::empty({n}, cov_2d.options());
    check_rc(gsr_screen_radii((int)n, cfp(cov_2d), fp(radii), current_stream()), "screen_radii");
    return radii;
}

// The glue's forward head in one kernel (rasterize.py:42-54): (mean_2d,
// cov_2d, depths, radii, colors, camera_position, opacity), bit for bit those
// of camera_position, project, screen_radii and SH; with alpha_logits also
// the opacity t.sigmoid(alpha_logits) (rasterize.py:149), else an empty tensor.
std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor> project_sh(
    int total_gaussians, const Tensor mu3d, const Tensor q3d, const Tensor s3d,
    const Tensor camera_rotation, const Tensor camera_translation, float fx, float fy, float cx,
    float cy, const Tensor albedo_coeff, const Tensor illumination_coeff,
    const c10::optional<Tensor>& alpha_logits) {
    CHECK_INPUT_FP32(mu3d);
    CHECK_INPUT_FP32(q3d);
    CHECK_INPUT_FP32(s3d);
    CHECK_INPUT_FP32(camera_rotation);
    CHECK_INPUT_FP32(camera_translation);
    CHECK_INPUT_FP32(albedo_coeff);
    CHECK_INPUT_FP32(illumination_coeff);
    TORCH_CHECK(total_gaussians >= 0, "total_gaussians must be non-negative");
    const int64_t n = total_gaussians;
    check_numel(mu3d, 3 * n, "mu3d must hold N x 3 values");
    check_numel(q3d, 4 * n, "q3d must hold N x 4 values");
    check_numel(s3d, 3 * n, "s3d must hold N x 3 values");
    check_numel(camera_rotation, 9, "camera_rotation must hold 3 x 3 values");
    check_numel(camera_translation, 3, "camera_translation must hold 3 values");
    check_numel(albedo_coeff, 3 * n, "albedo_coeff must hold N x 3 values");
    check_numel(illumination_coeff, 45 * n, "illumination_coeff must hold N x 15 x 3 values");
    const bool logits = alpha_logits.has_value() && alpha_logits->defined();
    if (logits) {
        CHECK_INPUT_FP32(*alpha_logits);
        TORCH_CHECK(alpha_logits->numel() == n, "alpha_logits must have N elements");
    }
    c10::hip::HIPGuardMasqueradingAsCUDA guard(mu3d.device());
    auto options = torch::TensorOptions().dtype(torch::kFloat32).device(mu3d.device());
    Tensor opacity = logits ? torch::empty_like(*alpha_logits) : torch::empty({0}, options);
    Tensor mean_2d = torch::empty({n, 2}, options);
    Tensor cov_2d = torch::empty({n, 3}, options);
    Tensor depths = torch::empty({n}, options);
    Tensor radii = torch::empty({n}, options);
    Tensor colors = torch::empty({n, 3}, options);
    Tensor cam = torch::empty({3}, options);
    const Tensor q_al = aligned16(q3d);
    const Tensor k_al = aligned16(illumination_coeff);
    check_rc(gsr_project_sh(total_gaussians, cfp(mu3d), cfp(q_al), cfp(s3d), cfp(camera_rotation),
                            cfp(camera_translation), fx, fy, cx, cy, cfp(albedo_coeff),
                            cfp(k_al), fp(mean_2d), fp(cov_2d), fp(depths), fp(radii),
                            fp(colors), fp(cam), logits ? cfp(*alpha_logits) : nullptr,
                            logits ? fp(opacity) : nullptr, current_stream()),
             "project_sh");
    return {mean_2d, cov_2d, depths, radii, colors, cam, opacity};
}

Tensor camera_position(const Tensor camera_rotation, const Tensor camera_translation) {
    CHECK_INPUT_FP32(camera_rotation);
    CHECK_INPUT_FP32(camera_translation);
    check_numel(camera_rotation, 9, "camera_rotation must hold 3 x 3 values");
    check_numel(camera_translation, 3, "camera_translation must hold 3 values");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(camera_rotation.device());
    Tensor cam = torch::empty({3}, camera_rotation.options());
    check_rc(gsr_camera_position(cfp(camera_rotation), cfp(camera_translation), fp(cam),
                                 current_stream()),
             "camera_position");
    return cam;
}

// ---- SH (bindings.cpp:32-46 / SH.cu:95-131) ----
Tensor spherical_harmonics(int total_gaussians, const Tensor camera_position,
                           const Tensor mu_world, const Tensor albedo_coeff,
                           const Tensor illumination_coeff) {
    CHECK_INPUT_FP32(camera_position);
    CHECK_INPUT_FP32(mu_world);
    CHECK_INPUT_FP32(albedo_coeff);
    CHECK_INPUT_FP32(illumination_coeff);
    TORCH_CHECK(camera_position.numel() >= 3, "camera_position must have 3 elements");
    TORCH_CHECK(total_gaussians >= 0, "total_gaussians must be non-negative");
    const int64_t n = total_gaussians;
    check_numel(mu_world, 3 * n, "mu_world must hold N x 3 values");
    check_numel(albedo_coeff, 3 * n, "albedo_coeff must hold N x 3 values");
    check_numel(illumination_coeff, 45 * n, "illumination_coeff must hold N x 15 x 3 values");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(mu_world.device());
    auto options = torch::TensorOptions().dtype(torch::kFloat32).device(mu_world.device());
    Tensor colors = torch::empty({n, 3}, options);
    const Tensor k_al = aligned16(illumination_coeff);
    check_rc(gsr_sh(total_gaussians, cfp(camera_position), cfp(mu_world), cfp(albedo_coeff),
                    cfp(k_al), fp(colors), current_stream()),
             "SH");
    return colors;
}

// ---- rasterize (bindings.cpp:50-70 / rasterize.cu:284-487) ----
std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor, Tensor> rasterize_impl(
    int num_gaussians, const Tensor& depths, const Tensor& mean_2d, const Tensor& cov_2d,
    const Tensor& colors, const Tensor& alpha, int height, int width, bool want_keys,
    const Tensor* order = nullptr, const Tensor* tile_skip = nullptr) {
    TORCH_CHECK(height >= 0 && width >= 0, "height and width must be non-negative");
    auto device = mean_2d.device();
    auto float_options = torch::TensorOptions().dtype(torch::kFloat32).device(device);
    auto int_options = torch::TensorOptions().dtype(torch::kInt32).device(device);
    auto key_options = torch::TensorOptions().dtype(torch::kInt64).device(device);
    const int64_t tiles = (int64_t)((width + 15) / 16) * ((height + 15) / 16);
    auto empty_buffers = [&]() {
        return std::make_tuple(torch::zeros({height, width, 3}, float_options),
                               torch::empty({0}, int_options),
                               torch::zeros({tiles, 2}, int_options),
                               torch::ones({height, width}, float_options),
                               torch::zeros({height, width}, int_options),
                               torch::empty({0}, key_options));
    };
    if (num_gaussians == 0) return empty_buffers();

    CHECK_INPUT_FP32(depths);
    CHECK_INPUT_FP32(mean_2d);
    CHECK_INPUT_FP32(cov_2d);
    CHECK_INPUT_FP32(colors);
    CHECK_INPUT_FP32(alpha);
    TORCH_CHECK(num_gaussians > 0, "num_gaussians must be non-negative");
    TORCH_CHECK(mean_2d.dim() == 2 && mean_2d.size(0) == num_gaussians && mean_2d.size(1) == 2,
                "mean_2d must have shape (N, 2)");
    TORCH_CHECK(cov_2d.dim() == 2 && cov_2d.size(0) == num_gaussians && cov_2d.size(1) == 3,
                "cov_2d must have shape (N, 3) upper-triangular [a, b, c]");
    TORCH_CHECK(colors.dim() == 2 && colors.size(0) == num_gaussians && colors.size(1) == 3,
                "colors must have shape (N, 3)");
    TORCH_CHECK(depths.numel() == num_gaussians, "depths must have N elements");
    TORCH_CHECK(alpha.numel() == num_gaussians, "alpha must have N elements");
    if (order) {
        TORCH_CHECK(order->is_cuda() && order->device() == mean_2d.device(),
                    "order must be a CUDA tensor on mean_2d's device");
        TORCH_CHECK(order->is_contiguous(), "order must be contiguous");
        TORCH_CHECK(order->scalar_type() == torch::kInt32 && order->numel() == num_gaussians,
                    "order must be an int32 tensor of N elements");
    }
    if (tile_skip) {
        TORCH_CHECK(tile_skip->is_cuda() && tile_skip->device() == mean_2d.device(),
                    "tile_skip must be a CUDA tensor on mean_2d's device");
        TORCH_CHECK(tile_skip->is_contiguous() && tile_skip->numel() == tiles &&
                        (tile_skip->scalar_type() == torch::kUInt8 ||
                         tile_skip->scalar_type() == torch::kBool),
                    "tile_skip must be a contiguous uint8 or bool tensor of one entry per tile");
    }

    c10::hip::HIPGuardMasqueradingAsCUDA guard(device);
    void* st = current_stream();
    Tensor bin_ws = workspace((int64_t)gsr_bin_workspace_bytes(num_gaussians, height, width),
                              mean_2d);
    int64_t m = 0;
    if (order)
        check_rc(gsr_rasterize_bin_ordered(num_gaussians, order->data_ptr<int32_t>(),
                                           cfp(mean_2d), cfp(cov_2d), height, width,
                                           bin_ws.data_ptr(), (size_t)bin_ws.numel(), &m, st),
                 "rasterize_ordered");
    else
        check_rc(gsr_rasterize_bin(num_gaussians, cfp(depths), cfp(mean_2d), cfp(cov_2d), height,
                                   width, bin_ws.data_ptr(), (size_t)bin_ws.numel(), &m, st),
                 "rasterize");
    if (m == 0) return empty_buffers();

    Tensor sort_ws = workspace(
        (int64_t)gsr_sort_workspace_bytes(m, num_gaussians, height, width), mean_2d);
    Tensor sorted_ids = torch::empty({m}, int_options);
    Tensor tile_ranges = torch::empty({tiles, 2}, int_options);
    Tensor rendered_img = torch::empty({height, width, 3}, float_options);
    Tensor final_T = torch::empty({height, width}, float_options);
    Tensor n_contrib = torch::empty({height, width}, int_options);
    Tensor sorted_keys = want_keys ? torch::empty({m}, key_options) : torch::empty({0}, key_options);
    if (tile_skip) {
        check_rc(gsr_rasterize_render_skip(
                     num_gaussians, cfp(depths), cfp(mean_2d), cfp(cov_2d), cfp(colors),
                     cfp(alpha), height, width, bin_ws.data_ptr(), (size_t)bin_ws.numel(), m,
                     sort_ws.data_ptr(), (size_t)sort_ws.numel(),
                     static_cast<const uint8_t*>(tile_skip->data_ptr()),
                     sorted_ids.data_ptr<int32_t>(), tile_ranges.data_ptr<int32_t>(),
                     fp(rendered_img), fp(final_T), n_contrib.data_ptr<int32_t>(), st),
                 "rasterize_ordered");
        return {rendered_img, sorted_ids, tile_ranges, final_T, n_contrib, sorted_keys};
    }
    check_rc(gsr_rasterize_render(
                 num_gaussians, cfp(depths), cfp(mean_2d), cfp(cov_2d), cfp(colors), cfp(alpha),
                 height, width, bin_ws.data_ptr(), (size_t)bin_ws.numel(), m,
                 sort_ws.data_ptr(), (size_t)sort_ws.numel(), sorted_ids.data_ptr<int32_t>(),
                 tile_ranges.data_ptr<int32_t>(), fp(rendered_img), fp(final_T),
                 n_contrib.data_ptr<int32_t>(),
                 want_keys ? reinterpret_cast<uint64_t*>(sorted_keys.data_ptr<int64_t>()) : nullptr,
                 st),
             "rasterize");
    return {rendered_img, sorted_ids, tile_ranges, final_T, n_contrib, sorted_keys};
}

std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor> rasterize(int num_gaussians,
                                                             const Tensor depths,
                                                             const Tensor mean_2d,
                                                             const Tensor cov_2d,
                                                             const Tensor colors,
                                                             const Tensor alpha, int height,
                                                             int width) {
    auto r = rasterize_impl(num_gaussians, depths, mean_2d, cov_2d, colors, alpha, height, width,
                            false);
    return {std::get<0>(r), std::get<1>(r), std::get<2>(r), std::get<3>(r), std::get<4>(r)};
}

// Not in the reference surface: `rasterize` plus the 64-bit sorted keys
// (tile << 32 | depth bits) the reference sorts internally, for bit-exact
// parity checks of the sort.
std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor, Tensor> rasterize_with_keys(
    int num_gaussians, const Tensor depths, const Tensor mean_2d, const Tensor cov_2d,
    const Tensor colors, const Tensor alpha, int height, int width) {
    return rasterize_impl(num_gaussians, depths, mean_2d, cov_2d, colors, alpha, height, width,
                          true);
}

// Not in the reference surface: every Gaussian stably sorted by the float bits
// of its depth (int32 [N]), shared by the screen bands of one frame.
Tensor depth_order(int num_gaussians, const Tensor& depths) {
    CHECK_INPUT_FP32(depths);
    TORCH_CHECK(num_gaussians >= 0 && depths.numel() == num_gaussians,
                "depths must have N elements");
    auto int_options = torch::TensorOptions().dtype(torch::kInt32).device(depths.device());
    Tensor order = torch::empty({num_gaussians}, int_options);
    if (num_gaussians == 0) return order;
    c10::hip::HIPGuardMasqueradingAsCUDA guard(depths.device());
    Tensor ws = workspace((int64_t)gsr_depth_order_workspace_bytes(num_gaussians), depths);
    check_rc(gsr_depth_order(num_gaussians, cfp(depths), ws.data_ptr(), (size_t)ws.numel(),
                             order.data_ptr<int32_t>(), current_stream()),
             "depth_order");
    return order;
}

// Not in the reference surface: `rasterize` with the depth order given (from
// depth_order) instead of sorted per call; with tile_skip (one uint8 or bool
// per tile) the lists of the marked tiles may be left empty
// (gsr_rasterize_render_skip).
std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor> rasterize_ordered(
    int num_gaussians, const Tensor order, const Tensor depths, const Tensor mean_2d,
    const Tensor cov_2d, const Tensor colors, const Tensor alpha, int height, int width,
    const c10::optional<Tensor>& tile_skip) {
    auto r = rasterize_impl(num_gaussians, depths, mean_2d, cov_2d, colors, alpha, height, width,
                            false, &order, tile_skip.has_value() ? &*tile_skip : nullptr);
    return {std::get<0>(r), std::get<1>(r), std::get<2>(r), std::get<3>(r), std::get<4>(r)};
}

// ---- backwards_rasterization (bindings.cpp:72-100 / rasterize_backward.cu:239-309) ----
// strided: grad_output is any [H, W, 3] fp32 view (the glue's variant, no
// counterpart in the reference, which requires it contiguous).
std::tuple<Tensor, Tensor, Tensor, Tensor> backwards_rasterization_impl(
    const Tensor& grad_output, const Tensor& mean_2d, const Tensor& cov_2d, const Tensor& colors,
    const Tensor& alpha, const Tensor& sorted_ids, const Tensor& tile_ranges,
    const Tensor& final_T, const Tensor& n_contrib, int num_gaussians, int height, int width,
    bool strided, const std::vector<Tensor>* accumulate = nullptr) {
    if (strided) {
        CHECK_CUDA(grad_output);
        CHECK_FP32(grad_output);
        TORCH_CHECK(grad_output.dim() == 3 && grad_output.size(0) == height &&
                        grad_output.size(1) == width && grad_output.size(2) == 3,
                    "grad_output must have shape (H, W, 3)");
    } else {
        CHECK_INPUT_FP32(grad_output);
    }
    CHECK_INPUT_FP32(mean_2d);
    CHECK_INPUT_FP32(cov_2d);
    CHECK_INPUT_FP32(colors);
    CHECK_INPUT_FP32(alpha);
    CHECK_INPUT_FP32(final_T);
    CHECK_INPUT_INT32(sorted_ids);
    CHECK_INPUT_INT32(tile_ranges);
    CHECK_INPUT_INT32(n_contrib);
    TORCH_CHECK(mean_2d.dim() == 2 && mean_2d.size(0) == num_gaussians && mean_2d.size(1) == 2,
                "mean_2d must have shape (N, 2)");
    TORCH_CHECK(cov_2d.dim() == 2 && cov_2d.size(0) == num_gaussians && cov_2d.size(1) == 3,
                "cov_2d must have shape (N, 3)");
    TORCH_CHECK(colors.dim() == 2 && colors.size(0) == num_gaussians && colors.size(1) == 3,
                "colors must have shape (N, 3)");
    TORCH_CHECK(alpha.numel() == num_gaussians, "alpha must have N elements");
    TORCH_CHECK(final_T.numel() == (int64_t)height * width, "final_T must have H*W elements");
    TORCH_CHECK(n_contrib.numel() == (int64_t)height * width, "n_contrib must have H*W elements");
    TORCH_CHECK(grad_output.numel() == (int64_t)height * width * 3,
                "grad_output must have H*W*3 elements");
    const int64_t tiles = (int64_t)((width + 15) / 16) * ((height + 15) / 16);
    TORCH_CHECK(tile_ranges.numel() >= 2 * tiles, "tile_ranges must have T x 2 elements");

    c10::hip::HIPGuardMasqueradingAsCUDA guard(mean_2d.device());
    auto options = torch::TensorOptions().dtype(torch::kFloat32).device(mean_2d.device());
    Tensor grad_mean_2d, grad_cov_2d, grad_colors, grad_alpha;
    if (accumulate) {
        TORCH_CHECK(accumulate->size() == 4, "accumulate_into must hold 4 tensors");
        const int64_t widths[4] = {2, 3, 3, 1};
        for (int k = 0; k < 4; ++k) {
            const Tensor& a = (*accumulate)[k];
            CHECK_INPUT_FP32(a);
            TORCH_CHECK(a.numel() == widths[k] * num_gaussians && a.device() == mean_2d.device(),
                        "accumulate_into tensors must be d mean2d [N,2], d cov2d [N,3], "
                        "d colors [N,3], d alpha [N,1] on the inputs' device");
        }
        grad_mean_2d = (*accumulate)[0];
        grad_cov_2d = (*accumulate)[1];
        grad_colors = (*accumulate)[2];
        grad_alpha = (*accumulate)[3];
    } else {
        grad_mean_2d = torch::empty({num_gaussians, 2}, options);
        grad_cov_2d = torch::empty({num_gaussians, 3}, options);
        grad_colors = torch::empty({num_gaussians, 3}, options);
        grad_alpha = torch::empty({num_gaussians, 1}, options);
    }
    Tensor ws =
        workspace((int64_t)gsr_backward_workspace_bytes(num_gaussians, sorted_ids.numel(),
                                                         height, width),
                  mean_2d);
    if (accumulate) {
        check_rc(gsr_rasterize_backward_accumulate(
                     num_gaussians, height, width, cfp(grad_output), grad_output.stride(0),
                     grad_output.stride(1), grad_output.stride(2), cfp(mean_2d), cfp(cov_2d),
                     cfp(colors), cfp(alpha), sorted_ids.data_ptr<int32_t>(), sorted_ids.numel(),
                     tile_ranges.data_ptr<int32_t>(), cfp(final_T),
                     n_contrib.data_ptr<int32_t>(), ws.data_ptr(), (size_t)ws.numel(),
                     fp(grad_mean_2d), fp(grad_cov_2d), fp(grad_colors), fp(grad_alpha),
                     current_stream()),
                 "backwards_rasterization_accumulate");
    } else if (strided) {
        check_rc(gsr_rasterize_backward_strided(
                     num_gaussians, height, width, cfp(grad_output), grad_output.stride(0),
                     grad_output.stride(1), grad_output.stride(2), cfp(mean_2d), cfp(cov_2d),
                     cfp(colors), cfp(alpha), sorted_ids.data_ptr<int32_t>(), sorted_ids.numel(),
                     tile_ranges.data_ptr<int32_t>(), cfp(final_T),
                     n_contrib.data_ptr<int32_t>(), ws.data_ptr(), (size_t)ws.numel(),
                     fp(grad_mean_2d), fp(grad_cov_2d), fp(grad_colors), fp(grad_alpha),
                     current_stream()),
                 "backwards_rasterization_strided");
    } else {
        check_rc(gsr_rasterize_backward(
                     num_gaussians, height, width, cfp(grad_output), cfp(mean_2d), cfp(cov_2d),
                     cfp(colors), cfp(alpha), sorted_ids.data_ptr<int32_t>(), sorted_ids.numel(),
                     tile_ranges.data_ptr<int32_t>(), cfp(final_T),
                     n_contrib.data_ptr<int32_t>(), ws.data_ptr(), (size_t)ws.numel(),
                     fp(grad_mean_2d), fp(grad_cov_2d), fp(grad_colors), fp(grad_alpha),
                     current_stream()),
                 "backwards_rasterization");
    }
    return {grad_mean_2d, grad_cov_2d, grad_colors, grad_alpha};
}

std::tuple<Tensor, Tensor, Tensor, Tensor> backwards_rasterization(
    const Tensor grad_output, const Tensor mean_2d, const Tensor cov_2d, const Tensor colors,
    const Tensor alpha, const Tensor sorted_ids, const Tensor tile_ranges, const Tensor final_T,
    const Tensor n_contrib, int num_gaussians, int height, int width) {
    return backwards_rasterization_impl(grad_output, mean_2d, cov_2d, colors, alpha, sorted_ids,
                                        tile_ranges, final_T, n_contrib, num_gaussians, height,
                                        width, false);
}

std::tuple<Tensor, Tensor, Tensor, Tensor> backwards_rasterization_strided(
    const Tensor grad_output, const Tensor mean_2d, const Tensor cov_2d, const Tensor colors,
    const Tensor alpha, const Tensor sorted_ids, const Tensor tile_ranges, const Tensor final_T,
    const Tensor n_contrib, int num_gaussians, int height, int width) {
    return backwards_rasterization_impl(grad_output, mean_2d, cov_2d, colors, alpha, sorted_ids,
                                        tile_ranges, final_T, n_contrib, num_gaussians, height,
                                        width, true);
}

// strided, adding into the four given gradient tensors (screen bands)
std::tuple<Tensor, Tensor, Tensor, Tensor> backwards_rasterization_accumulate(
    const Tensor grad_output, const Tensor mean_2d, const Tensor cov_2d, const Tensor colors,
    const Tensor alpha, const Tensor sorted_ids, const Tensor tile_ranges, const Tensor final_T,
    const Tensor n_contrib, int num_gaussians, int height, int width,
    std::vector<Tensor> accumulate_into) {
    return backwards_rasterization_impl(grad_output, mean_2d, cov_2d, colors, alpha, sorted_ids,
                                        tile_ranges, final_T, n_contrib, num_gaussians, height,
                                        width, true, &accumulate_into);
}

// ---- backwards_SH (bindings.cpp:102-116 / delight_backward.cu:176-218) ----
std::tuple<Tensor, Tensor, Tensor> backwards_SH(const Tensor colors_grad, const Tensor mu,
                                                const Tensor albedo, const Tensor k_j,
                                                const Tensor camera_position) {
    CHECK_INPUT_FP32(colors_grad);
    CHECK_INPUT_FP32(mu);
    CHECK_INPUT_FP32(albedo);
    CHECK_INPUT_FP32(k_j);
    CHECK_INPUT_FP32(camera_position);
    TORCH_CHECK(camera_position.numel() >= 3, "camera_position must have 3 elements");
    const int64_t n = mu.size(0);
    check_numel(colors_grad, 3 * n, "colors_grad must hold N x 3 values");
    check_numel(albedo, 3 * n, "albedo must hold N x 3 values");
    check_numel(k_j, 45 * n, "k_j must hold N x 15 x 3 values");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(mu.device());
    auto options = torch::TensorOptions().dtype(torch::kFloat32).device(mu.device());
    Tensor albedo_grad = torch::empty({n, 3}, options);
    Tensor k_j_grad = torch::empty({n, 15, 3}, options);
    Tensor mu_grad = torch::empty({n, 3}, options);
    const Tensor k_al = aligned16(k_j);
    check_rc(gsr_sh_backward((int)n, cfp(colors_grad), cfp(mu), cfp(albedo), cfp(k_al),
                             cfp(camera_position), fp(albedo_grad), fp(k_j_grad), fp(mu_grad),
                             current_stream()),
             "backwards_SH");
    return {albedo_grad, k_j_grad, mu_grad};
}

// ---- backwards_projection (bindings.cpp:118-138 / projection_backward.cu:142-187) ----
std::tuple<Tensor, Tensor, Tensor> backwards_projection(
    const Tensor mean_2d_grad, const Tensor cov_2d_grad, const Tensor mu, const Tensor q,
    const Tensor s, const Tensor camera_rotation, const Tensor camera_translation, float fx,
    float fy, float cx, float cy) {
    CHECK_INPUT_FP32(mean_2d_grad);
    CHECK_INPUT_FP32(cov_2d_grad);
    CHECK_INPUT_FP32(mu);
    CHECK_INPUT_FP32(q);
    CHECK_INPUT_FP32(s);
    CHECK_INPUT_FP32(camera_rotation);
    CHECK_INPUT_FP32(camera_translation);
    const int64_t n = mu.size(0);
    check_numel(mean_2d_grad, 2 * n, "mean_2d_grad must hold N x 2 values");
    check_numel(cov_2d_grad, 3 * n, "cov_2d_grad must hold N x 3 values");
    check_numel(q, 4 * n, "q must hold N x 4 values");
    check_numel(s, 3 * n, "s must hold N x 3 values");
    check_numel(camera_rotation, 9, "camera_rotation must hold 3 x 3 values");
    check_numel(camera_translation, 3, "camera_translation must hold 3 values");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(mu.device());
    auto options = torch::TensorOptions().dtype(torch::kFloat32).device(mu.device());
    Tensor mu_grad = torch::empty({n, 3}, options);
    Tensor q_grad = torch::empty({n, 4}, options);
    Tensor s_grad = torch::empty({n, 3}, options);
    const Tensor q_al = aligned16(q);
    check_rc(gsr_project_backward((int)n, cfp(mean_2d_grad), cfp(cov_2d_grad), cfp(mu), cfp(q_al),
                                  cfp(s), cfp(camera_rotation), cfp(camera_translation), fx, fy,
                                  cx, cy, fp(mu_grad), fp(q_grad), fp(s_grad), current_stream()),
             "backwards_projection");
    return {mu_grad, q_grad, s_grad};
}

// The glue's backward tail in one kernel (rasterize.py:100-117): (mu_grad,
// q_grad, s_grad, albedo_grad, k_j_grad, alpha_logits_grad) with mu_grad =
// the projection's + the SH's, bit for bit backwards_SH, backwards_projection
// and that sum; with alpha_grad and opacity also torch's sigmoid backward
// into alpha_logits_grad (shaped like opacity), else an empty tensor.
std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor, Tensor> backwards_project_sh(
    const Tensor mean_2d_grad, const Tensor cov_2d_grad, const Tensor colors_grad,
    const Tensor mu, const Tensor q, const Tensor s, const Tensor camera_rotation,
    const Tensor camera_translation, float fx, float fy, const Tensor albedo, const Tensor k_j,
    const Tensor camera_position, const c10::optional<Tensor>& alpha_grad,
    const c10::optional<Tensor>& opacity) {
    CHECK_INPUT_FP32(mean_2d_grad);
    CHECK_INPUT_FP32(cov_2d_grad);
    CHECK_INPUT_FP32(colors_grad);
    CHECK_INPUT_FP32(mu);
    CHECK_INPUT_FP32(q);
    CHECK_INPUT_FP32(s);
    CHECK_INPUT_FP32(camera_rotation);
    CHECK_INPUT_FP32(camera_translation);
    CHECK_INPUT_FP32(albedo);
    CHECK_INPUT_FP32(k_j);
    CHECK_INPUT_FP32(camera_position);
    const int64_t n = mu.size(0);
    check_numel(mean_2d_grad, 2 * n, "mean_2d_grad must hold N x 2 values");
    check_numel(cov_2d_grad, 3 * n, "cov_2d_grad must hold N x 3 values");
    check_numel(colors_grad, 3 * n, "colors_grad must hold N x 3 values");
    check_numel(q, 4 * n, "q must hold N x 4 values");
    check_numel(s, 3 * n, "s must hold N x 3 values");
    check_numel(camera_rotation, 9, "camera_rotation must hold 3 x 3 values");
    check_numel(camera_translation, 3, "camera_translation must hold 3 values");
    check_numel(albedo, 3 * n, "albedo must hold N x 3 values");
    check_numel(k_j, 45 * n, "k_j must hold N x 15 x 3 values");
    TORCH_CHECK(camera_position.numel() >= 3, "camera_position must have 3 elements");
    const bool sig = alpha_grad.has_value() && alpha_grad->defined();
    TORCH_CHECK(sig == (opacity.has_value() && opacity->defined()),
                "alpha_grad and opacity go together");
    if (sig) {
        CHECK_INPUT_FP32(*alpha_grad);
        CHECK_INPUT_FP32(*opacity);
        TORCH_CHECK(alpha_grad->numel() == n && opacity->numel() == n,
                    "alpha_grad and opacity must have N elements");
    }
    c10::hip::HIPGuardMasqueradingAsCUDA guard(mu.device());
    auto options = torch::TensorOptions().dtype(torch::kFloat32).device(mu.device());
    Tensor logit_grad = sig ? torch::empty_like(*opacity) : torch::empty({0}, options);
    Tensor mu_grad = torch::empty({n, 3}, options);
    Tensor q_grad = torch::empty({n, 4}, options);
    Tensor s_grad = torch::empty({n, 3}, options);
    Tensor albedo_grad = torch::empty({n, 3}, options);
    Tensor k_j_grad = torch::empty({n, 15, 3}, options);
    const Tensor q_al = aligned16(q);
    const Tensor k_al = aligned16(k_j);
    check_rc(gsr_project_sh_backward((int)n, cfp(mean_2d_grad), cfp(cov_2d_grad),
                                     cfp(colors_grad), cfp(mu), cfp(q_al), cfp(s),
                                     cfp(camera_rotation), cfp(camera_translation), fx, fy,
                                     cfp(albedo), cfp(k_al), cfp(camera_position), fp(mu_grad),
                                     fp(q_grad), fp(s_grad), fp(albedo_grad), fp(k_j_grad),
                                     sig ? cfp(*alpha_grad) : nullptr,
                                     sig ? cfp(*opacity) : nullptr,
                                     sig ? fp(logit_grad) : nullptr, current_stream()),
             "backwards_project_sh");
    return {mu_grad, q_grad, s_grad, albedo_grad, k_j_grad, logit_grad};
}

// ---- the trainer's loss (gaussian_splatting/utils/loss.py:12-33) ----
void check_image_pair(const Tensor& a, const Tensor& b, const char* an, const char* bn) {
    CHECK_INPUT_FP32(a);
    CHECK_INPUT_FP32(b);
    TORCH_CHECK(a.dim() == 3 && a.size(2) == 3, an, " must have shape (H, W, 3)");
    TORCH_CHECK(a.sizes() == b.sizes(), "Shape mismatch: gt ", b.sizes(), " vs rendered ",
                a.sizes());
    (void)bn;
}

// (out, ws): out = [loss, SSIM, L1 mean] on the device; ws feeds the backward.
std::tuple<Tensor, Tensor> l1_dssim(const Tensor rendered, const Tensor gt, double lambda_dssim) {
    check_image_pair(rendered, gt, "rendered", "gt");
    const int H = (int)rendered.size(0), W = (int)rendered.size(1);
    c10::hip::HIPGuardMasqueradingAsCUDA guard(rendered.device());
    Tensor ws = workspace((int64_t)gsr_loss_workspace_bytes(H, W), rendered);
    Tensor out = torch::empty({3}, rendered.options());
    check_rc(gsr_l1_dssim(H, W, cfp(rendered), cfp(gt), (float)lambda_dssim, ws.data_ptr(),
                          (size_t)ws.numel(), fp(out), current_stream()),
             "l1_dssim");
    return {out, ws};
}

Tensor l1_dssim_backward(const Tensor rendered, const Tensor gt, double lambda_dssim,
                         const Tensor ws, const c10::optional<Tensor>& grad_loss) {
    check_image_pair(rendered, gt, "rendered", "gt");
    const int H = (int)rendered.size(0), W = (int)rendered.size(1);
    const bool g = grad_loss.has_value() && grad_loss->defined();
    if (g) {
        CHECK_INPUT_FP32(*grad_loss);
        TORCH_CHECK(grad_loss->numel() == 1, "grad_loss must hold one value");
    }
    TORCH_CHECK(ws.is_cuda() && ws.scalar_type() == torch::kUInt8, "ws must be the forward's");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(rendered.device());
    Tensor d = torch::empty_like(rendered);
    check_rc(gsr_l1_dssim_backward(H, W, cfp(rendered), cfp(gt), (float)lambda_dssim,
                                   ws.data_ptr(), (size_t)ws.numel(), g ? cfp(*grad_loss) : nullptr,
                                   fp(d), current_stream()),
             "l1_dssim_backward");
    return d;
}

// [1 - SSIM, SSIM, mean|a - b|] on the device (scripts/eval.py:60)
Tensor ssim(const Tensor a, const Tensor b) {
    check_image_pair(a, b, "a", "b");
    const int H = (int)a.size(0), W = (int)a.size(1);
    c10::hip::HIPGuardMasqueradingAsCUDA guard(a.device());
    Tensor ws = workspace((int64_t)gsr_loss_workspace_bytes(H, W), a);
    Tensor out = torch::empty({3}, a.options());
    check_rc(gsr_ssim(H, W, cfp(a), cfp(b), ws.data_ptr(), (size_t)ws.numel(), fp(out),
                      current_stream()),
             "ssim");
    return out;
}

// ---- the trainer's optimizer step (utils/optim.py:12-31, train.py:171-176) ----
void adam_step(const std::vector<Tensor>& params, const std::vector<Tensor>& grads,
               const std::vector<Tensor>& exp_avgs, const std::vector<Tensor>& exp_avg_sqs,
               const std::vector<double>& lrs, const std::vector<int64_t>& steps,
               const std::vector<double>& clamp_min, const std::vector<double>& clamp_max,
               double beta1, double beta2, double eps) {
    const size_t n = params.size();
    TORCH_CHECK(grads.size() == n && exp_avgs.size() == n && exp_avg_sqs.size() == n &&
                    lrs.size() == n && steps.size() == n && clamp_min.size() == n &&
                    clamp_max.size() == n,
                "adam_step: one gradient, state pair, lr, step and clamp pair per parameter");
    if (n == 0) return;
    std::vector<gsr_adam_tensor> t(n);
    for (size_t i = 0; i < n; ++i) {
        const Tensor& p = params[i];
        CHECK_INPUT_FP32(p);
        CHECK_INPUT_FP32(grads[i]);
        CHECK_INPUT_FP32(exp_avgs[i]);
        CHECK_INPUT_FP32(exp_avg_sqs[i]);
        TORCH_CHECK(grads[i].numel() == p.numel() && exp_avgs[i].numel() == p.numel() &&
                        exp_avg_sqs[i].numel() == p.numel(),
                    "adam_step: gradient and state must match the parameter's size");
        TORCH_CHECK(grads[i].device() == p.device() && exp_avgs[i].device() == p.device() &&
                        exp_avg_sqs[i].device() == p.device() &&
                        p.device() == params[0].device(),
                    "adam_step: all tensors must be on one device");
        t[i] = gsr_adam_tensor{fp(p),         cfp(grads[i]), fp(exp_avgs[i]), fp(exp_avg_sqs[i]),
                               p.numel(),     lrs[i],        steps[i],        (float)clamp_min[i],
                               (float)clamp_max[i]};
    }
    c10::hip::HIPGuardMasqueradingAsCUDA guard(params[0].device());
    check_rc(gsr_adam_step((int)n, t.data(), beta1, beta2, eps, current_stream()), "adam_step");
}

// ---- the PLY export's vertex records (scripts/run.py:66-165) ----
Tensor ply_records(const Tensor mu, const Tensor q, const Tensor s, const Tensor alpha,
                   const Tensor albedo, const Tensor k_j, bool opacity_from_probability) {
    CHECK_INPUT_FP32(mu);
    CHECK_INPUT_FP32(q);
    CHECK_INPUT_FP32(s);
    CHECK_INPUT_FP32(alpha);
    CHECK_INPUT_FP32(albedo);
    CHECK_INPUT_FP32(k_j);
    const int64_t n = mu.size(0);
    TORCH_CHECK(k_j.dim() == 3 && k_j.size(0) == n && k_j.size(2) == 3,
                "Expected k_j shape (N, K, 3), got ", k_j.sizes());
    const int64_t K = k_j.size(1);
    check_numel(mu, 3 * n, "mu must hold N x 3 values");
    check_numel(q, 4 * n, "q must hold N x 4 values");
    check_numel(s, 3 * n, "s must hold N x 3 values");
    check_numel(alpha, n, "alpha must hold N values");
    check_numel(albedo, 3 * n, "albedo must hold N x 3 values");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(mu.device());
    Tensor out = torch::empty({n, 17 + 3 * K}, mu.options());
    const Tensor q_al = aligned16(q);
    check_rc(gsr_ply_pack((int)n, (int)K, cfp(mu), cfp(q_al), cfp(s), cfp(alpha), cfp(albedo),
                          cfp(k_j), opacity_from_probability ? 1 : 0, fp(out), current_stream()),
             "ply_records");
    return out;
}

// ---- adaptive density control (gaussian_splatting/utils/adc.py) ----
void adc_stats(const c10::optional<Tensor>& mean2d_grad, int width, int height,
               const c10::optional<Tensor>& radii, const Tensor grad_accum, const Tensor denom,
               const Tensor max_radii2d) {
    CHECK_INPUT_FP32(grad_accum);
    CHECK_INPUT_FP32(denom);
    CHECK_INPUT_FP32(max_radii2d);
    const int64_t n = grad_accum.numel();
    TORCH_CHECK(denom.numel() == n && max_radii2d.numel() == n,
                "densification buffers must have N elements");
    const bool g = mean2d_grad.has_value() && mean2d_grad->defined();
    const bool r = radii.has_value() && radii->defined();
    if (g) {
        CHECK_INPUT_FP32(*mean2d_grad);
        TORCH_CHECK(mean2d_grad->numel() == 2 * n, "mean2d_grad must have shape (N, 2)");
    }
    if (r) {
        CHECK_INPUT_FP32(*radii);
        TORCH_CHECK(radii->numel() == n, "radii must have N elements");
    }
    c10::hip::HIPGuardMasqueradingAsCUDA guard(grad_accum.device());
    check_rc(gsr_adc_stats((int)n, g ? cfp(*mean2d_grad) : nullptr, width, height,
                           r ? cfp(*radii) : nullptr, fp(grad_accum), fp(denom), fp(max_radii2d),
                           current_stream()),
             "adc_stats");
}

gsr_adc_config adc_cfg(double grad_threshold, double percent_dense, double scene_extent,
                       double min_opacity, c10::optional<double> max_screen_size, bool densify,
                       bool prune, bool reset_opacity) {
    gsr_adc_config c;
    c.grad_threshold = grad_threshold;
    c.percent_dense = percent_dense;
    c.scene_extent = scene_extent;
    c.min_opacity = min_opacity;
    c.has_max_screen_size = max_screen_size.has_value() ? 1 : 0;
    c.max_screen_size = max_screen_size.value_or(0.0);
    c.densify = densify ? 1 : 0;
    c.prune = prune ? 1 : 0;
    c.reset_opacity = reset_opacity ? 1 : 0;
    return c;
}

const int64_t kAdcWidths[6] = {3, 4, 3, 1, 3, 45};

void check_cloud(const std::vector<Tensor>& p, int64_t n) {
    TORCH_CHECK(p.size() == 6, "the cloud is six tensors: mu, q, s, alpha, A, k_j");
    for (int a = 0; a < 6; ++a) {
        CHECK_INPUT_FP32(p[a]);
        TORCH_CHECK(p[a].numel() == n * kAdcWidths[a], "cloud tensor ", a, " must hold N x ",
                    kAdcWidths[a], " values");
    }
}

// (counts[5], ws): the plan of the densify / prune pass
std::tuple<std::vector<int64_t>, Tensor> adc_plan(
    const std::vector<Tensor>& params, const Tensor grad_accum, const Tensor denom,
    const c10::optional<Tensor>& max_radii2d, double grad_threshold, double percent_dense,
    double scene_extent, double min_opacity, c10::optional<double> max_screen_size,
    bool densify, bool prune, bool reset_opacity) {
    const int64_t n = params.empty() ? 0 : params[0].size(0);
    check_cloud(params, n);
    CHECK_INPUT_FP32(grad_accum);
    CHECK_INPUT_FP32(denom);
    TORCH_CHECK(grad_accum.numel() == n && denom.numel() == n,
                "densification buffers must have N elements");
    const bool r = max_radii2d.has_value() && max_radii2d->defined();
    if (r) {
        CHECK_INPUT_FP32(*max_radii2d);
        TORCH_CHECK(max_radii2d->numel() == n, "max_radii2D must have N elements");
    }
    c10::hip::HIPGuardMasqueradingAsCUDA guard(params[0].device());
    Tensor ws = workspace((int64_t)gsr_adc_workspace_bytes((int)n), params[0]);
    const gsr_adc_config c = adc_cfg(grad_threshold, percent_dense, scene_extent, min_opacity,
                                     max_screen_size, densify, prune, reset_opacity);
    float* pp[6];
    for (int a = 0; a < 6; ++a) pp[a] = fp(params[a]);
    std::vector<int64_t> counts(5, 0);
    check_rc(gsr_adc_plan((int)n, pp, cfp(grad_accum), cfp(denom),
                          r ? cfp(*max_radii2d) : nullptr, &c, ws.data_ptr(), (size_t)ws.numel(),
                          counts.data(), current_stream()),
             "adc_plan");
    return {counts, ws};
}

// the new cloud (6 tensors) and its moments (12, undefined where the input's are)
std::tuple<std::vector<Tensor>, std::vector<c10::optional<Tensor>>> adc_apply(
    const std::vector<Tensor>& params, const std::vector<c10::optional<Tensor>>& moments,
    const Tensor noise, const Tensor ws, int64_t n_out, double grad_threshold,
    double percent_dense, double scene_extent, double min_opacity,
    c10::optional<double> max_screen_size, bool densify, bool prune, bool reset_opacity) {
    const int64_t n = params.empty() ? 0 : params[0].size(0);
    check_cloud(params, n);
    TORCH_CHECK(moments.size() == 12, "moments: exp_avg of each tensor, then exp_avg_sq");
    CHECK_INPUT_FP32(noise);
    TORCH_CHECK(ws.is_cuda() && ws.scalar_type() == torch::kUInt8 &&
                    ws.numel() >= (int64_t)gsr_adc_workspace_bytes((int)n),
                "ws must be the plan's");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(params[0].device());
    std::vector<Tensor> out(6);
    std::vector<c10::optional<Tensor>> mout(12);
    float* pin[6];
    float* pout[6];
    float* min_[12];
    float* mo[12];
    for (int a = 0; a < 6; ++a) {
        std::vector<int64_t> shape = params[a].sizes().vec();
        shape[0] = n_out;
        out[a] = torch::empty(shape, params[a].options());
        pin[a] = fp(params[a]);
        pout[a] = fp(out[a]);
    }
    for (int a = 0; a < 12; ++a) {
        const auto& mt = moments[a];
        if (mt.has_value() && mt->defined()) {
            CHECK_INPUT_FP32(*mt);
            TORCH_CHECK(mt->numel() == n * kAdcWidths[a % 6], "moment ", a, " must match its tensor");
            min_[a] = fp(*mt);
            mout[a] = torch::empty(out[a % 6].sizes(), mt->options());
            mo[a] = fp(*mout[a]);
        } else {
            min_[a] = nullptr;
            mo[a] = nullptr;
        }
    }
    const gsr_adc_config c = adc_cfg(grad_threshold, percent_dense, scene_extent, min_opacity,
                                     max_screen_size, densify, prune, reset_opacity);
    if (n_out > 0)  // an empty new cloud has nothing to write
        check_rc(gsr_adc_apply((int)n, pin, min_, cfp(noise), &c, ws.data_ptr(),
                               (size_t)ws.numel(), pout, mo, current_stream()),
                 "adc_apply");
    return {out, mout};
}

}  // namespace

PYBIND11_MODULE(custom_rasterizer_cuda, m) {
    m.doc() = "MI355X (gfx950) Gaussian-splatting rasterizer behind the custom_rasterizer_cuda "
              "surface";
    m.def("project", &project, "3DGS projection (HIP, gfx950)");
    m.def("SH", &spherical_harmonics, "3DGS spherical harmonics (HIP, gfx950)");
    m.def("rasterize", &rasterize, "3DGS tile rasterization (HIP, gfx950)");
    m.def("backwards_rasterization", &backwards_rasterization,
          "3DGS backward rasterization (HIP, gfx950)");
    m.def("backwards_rasterization_strided", &backwards_rasterization_strided,
          "glue: backwards_rasterization with grad_output any (H, W, 3) view, no copy");
    m.def("backwards_rasterization_accumulate", &backwards_rasterization_accumulate,
          "glue: backwards_rasterization_strided adding into accumulate_into "
          "(d mean2d, d cov2d, d colors, d alpha) in place; returns them");
    m.def("backwards_SH", &backwards_SH, "3DGS backward spherical harmonics (HIP, gfx950)");
    m.def("backwards_projection", &backwards_projection,
          "3DGS backward projection (HIP, gfx950)");
    m.def("depth_order", &depth_order,
          "every Gaussian stably sorted by the float bits of its depth (int32 [N])");
    m.def("rasterize_ordered", &rasterize_ordered,
          "rasterize with a depth order from depth_order (screen bands of one frame); with "
          "tile_skip the lists of the marked tiles may be left empty",
          py::arg("num_gaussians"), py::arg("order"), py::arg("depths"), py::arg("mean_2d"),
          py::arg("cov_2d"), py::arg("colors"), py::arg("alpha"), py::arg("height"),
          py::arg("width"), py::arg("tile_skip") = py::none());
    m.def("rasterize_with_keys", &rasterize_with_keys,
          "rasterize, also returning the sorted 64-bit keys (tile << 32 | depth bits)");
    m.def("library_version", []() { return std::string(gsr_version()); });
    m.def("library_sources", []() { return std::string(gsr_build_sources()); });
    m.def("screen_radii", &screen_radii, "glue: approximate screen radii (one kernel)");
    m.def("camera_position", &camera_position, "glue: camera position -R^T t (one kernel)");
    m.def("project_sh", &project_sh,
          "glue: camera position, project, screen radii, SH (and the opacity sigmoid) in one "
          "kernel",
          py::arg("total_gaussians"), py::arg("mu3d"), py::arg("q3d"), py::arg("s3d"),
          py::arg("camera_rotation"), py::arg("camera_translation"), py::arg("fx"), py::arg("fy"),
          py::arg("cx"), py::arg("cy"), py::arg("albedo_coeff"), py::arg("illumination_coeff"),
          py::arg("alpha_logits") = py::none());
    m.def("backwards_project_sh", &backwards_project_sh,
          "glue: backwards_SH, backwards_projection, their dL/dmu sum (and the sigmoid's "
          "backward) in one kernel",
          py::arg("mean_2d_grad"), py::arg("cov_2d_grad"), py::arg("colors_grad"), py::arg("mu"),
          py::arg("q"), py::arg("s"), py::arg("camera_rotation"), py::arg("camera_translation"),
          py::arg("fx"), py::arg("fy"), py::arg("albedo"), py::arg("k_j"),
          py::arg("camera_position"), py::arg("alpha_grad") = py::none(),
          py::arg("opacity") = py::none());
    m.def("l1_dssim", &l1_dssim,
          "trainer loss (1 - l) L1 + l (1 - SSIM): (tensor [loss, SSIM, L1], workspace)");
    m.def("l1_dssim_backward", &l1_dssim_backward, "dloss/drendered, scaled by grad_loss",
          py::arg("rendered"), py::arg("gt"), py::arg("lambda_dssim"), py::arg("ws"),
          py::arg("grad_loss") = py::none());
    m.def("ssim", &ssim, "SSIM of two (H, W, 3) images: tensor [1 - SSIM, SSIM, L1]");
    m.def("ply_records", &ply_records,
          "Inria 3DGS PLY vertex records [N, 17 + 3K] of a Gaussian cloud (run.py:66-165)");
    m.def("adc_stats", &adc_stats, "densification statistics (adc.py:58-87)",
          py::arg("mean2d_grad"), py::arg("width"), py::arg("height"), py::arg("radii"),
          py::arg("grad_accum"), py::arg("denom"), py::arg("max_radii2d"));
    m.def("adc_plan", &adc_plan, "densify / prune plan: (counts[5], workspace)");
    m.def("adc_apply", &adc_apply, "densify / prune gather: (new cloud, new moments)");
    m.def("adam_step", &adam_step,
          "fused Adam step (torch.optim.Adam arithmetic) with per-tensor clamps, in place",
          py::arg("params"), py::arg("grads"), py::arg("exp_avgs"), py::arg("exp_avg_sqs"),
          py::arg("lrs"), py::arg("steps"), py::arg("clamp_min"), py::arg("clamp_max"),
          py::arg("beta1"), py::arg("beta2"), py::arg("eps"));
    // Stage timing of libgsraster (HIP events on the launch stream); not part of
    // the reference surface.
    m.def("profile_enable", [](bool on) { gsr_profile_enable(on ? 1 : 0); });
    m.def("profile_reset", []() { gsr_profile_reset(); });
    // pairs per tile row, for planning screen bands (no reference counterpart)
    m.def("tile_row_pairs", [](int64_t n, const Tensor& mean_2d, const Tensor& cov_2d,
                               int64_t height, int64_t width) {
        CHECK_INPUT_FP32(mean_2d);
        CHECK_INPUT_FP32(cov_2d);
        const int64_t ty = (height + 15) / 16;
        auto rows = torch::empty({ty + 1}, mean_2d.options().dtype(torch::kInt64));
        check_rc(gsr_tile_row_pairs((int)n, mean_2d.data_ptr<float>(), cov_2d.data_ptr<float>(),
                                    (int)height, (int)width,
                                    reinterpret_cast<uint64_t*>(rows.data_ptr<int64_t>()),
                                    current_stream()),
                 "tile_row_pairs");
        return rows.narrow(0, 0, ty);
    }, py::arg("n"), py::arg("mean_2d"), py::arg("cov_2d"), py::arg("height"), py::arg("width"));
    // the Gaussians whose tile rectangle (widened by a tile row each way) holds
    // a tile marked in tile_mask [ceil(H / 16), ceil(W / 16)] (no reference
    // counterpart: depth-prefix screen bands)
    m.def("tiles_touch", [](int64_t n, const Tensor& mean_2d, const Tensor& cov_2d,
                            int64_t height, int64_t width, const Tensor& tile_mask) {
        CHECK_INPUT_FP32(mean_2d);
        CHECK_INPUT_FP32(cov_2d);
        const int64_t ty = (height + 15) / 16, tx = (width + 15) / 16;
        TORCH_CHECK(tile_mask.is_cuda() && tile_mask.dim() == 2 && tile_mask.size(0) == ty &&
                        tile_mask.size(1) == tx,
                    "tile_mask must be a CUDA tensor of shape [ceil(H/16), ceil(W/16)]");
        TORCH_CHECK(mean_2d.size(0) >= n && cov_2d.size(0) >= n, "fewer than n Gaussians");
        auto sat = torch::constant_pad_nd(
                       tile_mask.to(torch::kInt32).cumsum(0, torch::kInt32).cumsum(1, torch::kInt32),
                       {1, 0, 1, 0}, 0)
                       .contiguous();
        auto flags = torch::empty({n}, mean_2d.options().dtype(torch::kUInt8));
        check_rc(gsr_tiles_touch((int)n, mean_2d.data_ptr<float>(), cov_2d.data_ptr<float>(),
                                 (int)height, (int)width, sat.data_ptr<int32_t>(),
                                 flags.data_ptr<uint8_t>(), current_stream()),
                 "tiles_touch");
        return flags.to(torch::kBool);
    }, py::arg("n"), py::arg("mean_2d"), py::arg("cov_2d"), py::arg("height"), py::arg("width"),
       py::arg("tile_mask"));
    // VALU issue-rate calibration kernels (measurement support for bench.py)
    m.def("calibrate_valu", [](int kind, int iters) {
        auto out = torch::empty({(int64_t)gsr_calibrate_valu_out_floats()},
                                torch::dtype(torch::kFloat32).device(torch::kCUDA));
        check_rc(gsr_calibrate_valu(kind, iters, out.data_ptr<float>(), current_stream()),
                 "calibrate_valu");
        return out;
    }, py::arg("kind"), py::arg("iters"));
    m.def("profile_collect", []() {
        check_rc(gsr_profile_collect(), "profile_collect");
        py::dict out;
        for (int i = 0;; ++i) {
            const char* st = gsr_profile_stage(i);
            if (!st) break;
            int64_t c = 0;
            double ms = 0.0;
            gsr_profile_get(st, &c, &ms);
            if (c) out[st] = py::make_tuple(c, ms);
        }
        return out;
    });
}

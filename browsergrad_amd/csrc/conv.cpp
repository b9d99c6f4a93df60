// C entry points of the convolutions: the reference bridge's conv1d / conv2d
// methods (realizer.ts:1153-1521) and bg_conv_ex, the descriptor form the
// plan executor lowers CONV1D*, CONV2D*, CONV3D* and CONV_TRANSPOSE2D* onto
// (tensor_plan.ts:554-641).  Validation follows validateConv1dShape /
// validateConv2dShape (realizer.ts:722-799): positive sizes, non-negative
// padding, channels divisible by groups; f32 only (assertF32).  The handles'
// element counts are checked against the described shapes as well, which the
// reference leaves to the caller.
#include <string>

#include "core.h"

using namespace bg;

namespace {

void positive(int64_t v, const std::string& op, const char* name) {
  if (v <= 0) fail(BG_E_INVALID, "HIP bridge: " + op + "." + name + " must be a positive integer");
}

void need_f32(int dtype, const std::string& op) {
  if (dtype != BG_F32)
    fail(BG_E_DTYPE, "HIP bridge: " + op + " supports float32 only, got " + dtype_name(dtype));
}

const Record& operand(bg_ctx* ctx, bg_handle h, int64_t want, const std::string& op, const char* role) {
  const Record& r = get(ctx, h, (op + "[" + role + "]").c_str());
  if (r.dtype != BG_F32)
    fail(BG_E_DTYPE, "HIP bridge: " + op + "[" + role + "] must be float32, got " + dtype_name(r.dtype));
  if (r.numel() != want)
    fail(BG_E_SHAPE, "HIP bridge: " + op + "[" + role + "] holds " + std::to_string(r.numel()) +
                         " elements, expected " + std::to_string(want));
  return r;
}

// The descriptor's spatial arrays as (D, H, W), unit-padded.
void spatial3(const int64_t* src, int spatial, int64_t fill, int64_t (&dst)[3]) {
  for (int i = 0; i < 3; ++i) dst[i] = fill;
  for (int i = 0; i < spatial; ++i) dst[3 - spatial + i] = src[i];
}

int64_t prod3(const int64_t (&v)[3]) { return v[0] * v[1] * v[2]; }

std::string op_name(const bg_conv_desc& d) {
  static const char* ops[4] = {"", "_backward_input", "_backward_weight", "_backward_bias"};
  std::string base = d.transposed ? "conv_transpose" : "conv";
  return base + std::to_string(d.spatial) + "d" + ops[d.op];
}

void validate(const bg_conv_desc& d, const std::string& op) {
  if (d.spatial < 1 || d.spatial > 3) fail(BG_E_INVALID, "HIP bridge: " + op + " spatial rank must be 1, 2 or 3");
  positive(d.n, op, "n");
  positive(d.c_in, op, "cIn");
  positive(d.c_out, op, "cOut");
  positive(d.groups, op, "groups");
  static const char* axes[3] = {"d", "h", "w"};
  for (int i = 0; i < d.spatial; ++i) {
    const std::string ax = d.spatial == 1 ? "" : axes[3 - d.spatial + i];
    positive(d.in[i], op, (d.spatial == 1 ? std::string("lIn") : ax).c_str());
    positive(d.out[i], op, (d.spatial == 1 ? std::string("lOut") : "out_" + ax).c_str());
    positive(d.k[i], op, (d.spatial == 1 ? std::string("k") : "k" + ax).c_str());
    positive(d.stride[i], op, (d.spatial == 1 ? std::string("stride") : "stride_" + ax).c_str());
    positive(d.dilation[i], op, (d.spatial == 1 ? std::string("dilation") : "dilation_" + ax).c_str());
    if (d.pad[i] < 0) fail(BG_E_INVALID, "HIP bridge: " + op + " padding must be non-negative integers");
    if (d.transposed && (d.output_pad[i] < 0 || d.output_pad[i] >= d.stride[i]))
      fail(BG_E_INVALID, "HIP bridge: " + op + " output_padding must be non-negative and smaller than stride");
  }
  if (d.c_in % d.groups != 0 || d.c_out % d.groups != 0)
    fail(BG_E_INVALID, "HIP bridge: " + op + " channels must be divisible by groups");
  if (d.groups > 65535) fail(BG_E_INVALID, "HIP bridge: " + op + " groups above 65535 are not supported");
}

// Runs one descriptor; returns the new handle.
bg_handle run_conv(bg_ctx* ctx, const bg_conv_desc& d) {
  const std::string op = op_name(d);
  validate(d, op);
  int64_t in3[3], out3[3], k3[3], s3[3], p3[3], dl3[3];
  spatial3(d.in, d.spatial, 1, in3);
  spatial3(d.out, d.spatial, 1, out3);
  spatial3(d.k, d.spatial, 1, k3);
  spatial3(d.stride, d.spatial, 1, s3);
  spatial3(d.pad, d.spatial, 0, p3);
  spatial3(d.dilation, d.spatial, 1, dl3);
  const int64_t S_in = prod3(in3), S_out = prod3(out3), KV = prod3(k3);
  const int64_t n = d.n, ci = d.c_in, co = d.c_out, G = d.groups;
  // Shapes of the user-facing tensors.
  std::vector<int64_t> x_shape{n, ci}, y_shape{n, co}, w_shape;
  for (int i = 0; i < d.spatial; ++i) x_shape.push_back(d.in[i]);
  for (int i = 0; i < d.spatial; ++i) y_shape.push_back(d.out[i]);
  if (d.transposed) w_shape = {ci, co / G};
  else w_shape = {co, ci / G};
  for (int i = 0; i < d.spatial; ++i) w_shape.push_back(d.k[i]);
  const int64_t x_n = n * ci * S_in, y_n = n * co * S_out, w_n = numel(w_shape);

  // Index spaces the kernels decompose in 32 bits.
  const int64_t lim = int64_t(1) << 31;
  for (int64_t v : {x_n / ci, y_n / co, n * S_in, n * S_out, (ci / G) * KV, (co / G) * KV, ci * S_in, co * S_out})
    if (v >= lim) fail(BG_E_INVALID, "HIP bridge: " + op + " is larger than this build's 2^31 index spaces");

  // The conv picture: x [n][c][in] -> y [n][o][out], weight [o][c/G][kv].
  ConvProblem p{};
  p.n = n;
  p.groups = G;
  for (int i = 0; i < 3; ++i) {
    p.k[i] = k3[i];
    p.stride[i] = s3[i];
    p.pad[i] = p3[i];
    p.dil[i] = dl3[i];
  }
  auto set_io = [&](int64_t c, const int64_t (&i3)[3], int64_t o, const int64_t (&o3)[3]) {
    p.c = c;
    p.o = o;
    for (int i = 0; i < 3; ++i) {
      p.in[i] = i3[i];
      p.out[i] = o3[i];
    }
  };
  if (!d.transposed) set_io(ci, in3, co, out3);
  else set_io(co, out3, ci, in3);  // the transposed op's output is the conv picture's input

  const int64_t flops = 2 * n * p.o * (p.out[0] * p.out[1] * p.out[2]) * (p.c / G) * KV;
  bg_handle result = 0;
  if (d.op == BG_CONV_FORWARD) {
    const Record& rx = operand(ctx, d.a, x_n, op, "input");
    const Record& rw = operand(ctx, d.b, w_n, op, "weight");
    const float* bias = nullptr;
    if (d.bias) bias = reinterpret_cast<const float*>(operand(ctx, d.bias, co, op, "bias").ptr());
    const float* px = reinterpret_cast<const float*>(rx.ptr());
    const float* pw = reinterpret_cast<const float*>(rw.ptr());
    result = mint(ctx, size_t(y_n) * 4, y_shape, BG_F32);
    float* py = reinterpret_cast<float*>(ctx->handles[result].ptr());
    Profile prof(ctx, op.c_str(), (x_n + w_n + y_n) * 4, flops);
    launch_conv(ctx, p, d.transposed ? 1 : 0, px, pw, bias, py);
  } else if (d.op == BG_CONV_BACKWARD_INPUT) {
    const Record& rdy = operand(ctx, d.a, y_n, op, "dy");
    const Record& rw = operand(ctx, d.b, w_n, op, "weight");
    const float* pdy = reinterpret_cast<const float*>(rdy.ptr());
    const float* pw = reinterpret_cast<const float*>(rw.ptr());
    result = mint(ctx, size_t(x_n) * 4, x_shape, BG_F32);
    float* px = reinterpret_cast<float*>(ctx->handles[result].ptr());
    Profile prof(ctx, op.c_str(), (x_n + w_n + y_n) * 4, flops);
    launch_conv(ctx, p, d.transposed ? 0 : 1, pdy, pw, nullptr, px);
  } else if (d.op == BG_CONV_BACKWARD_WEIGHT) {
    const Record& rdy = operand(ctx, d.a, y_n, op, "dy");
    const Record& rx = operand(ctx, d.b, x_n, op, "input");
    const float* pdy = reinterpret_cast<const float*>(rdy.ptr());
    const float* px = reinterpret_cast<const float*>(rx.ptr());
    result = mint(ctx, size_t(w_n) * 4, w_shape, BG_F32);
    float* pw = reinterpret_cast<float*>(ctx->handles[result].ptr());
    Profile prof(ctx, op.c_str(), (x_n + w_n + y_n) * 4, flops);
    // WGRAD takes the conv picture's (dy, x): for the transposed op those
    // are (x, dy).
    if (!d.transposed) launch_conv(ctx, p, 2, pdy, px, nullptr, pw);
    else launch_conv(ctx, p, 2, px, pdy, nullptr, pw);
  } else if (d.op == BG_CONV_BACKWARD_BIAS) {
    const Record& rdy = operand(ctx, d.a, y_n, op, "dy");
    const float* pdy = reinterpret_cast<const float*>(rdy.ptr());
    result = mint(ctx, size_t(co) * 4, {co}, BG_F32);
    float* pb = reinterpret_cast<float*>(ctx->handles[result].ptr());
    Profile prof(ctx, op.c_str(), (y_n + co) * 4, 0);
    launch_conv_bias_grad(ctx, pdy, pb, n, co, S_out);
  } else {
    fail(BG_E_INVALID, "HIP bridge: conv op " + std::to_string(d.op) + " is unknown");
  }
  return result;
}

bg_conv_desc desc1d(int op, bg_handle a, bg_handle b, bg_handle bias, int64_t n, int64_t c_in, int64_t l_in,
                    int64_t c_out, int64_t k, int64_t stride, int64_t padding, int64_t dilation, int64_t groups,
                    int64_t l_out) {
  bg_conv_desc d{};
  d.op = op;
  d.spatial = 1;
  d.n = n;
  d.c_in = c_in;
  d.c_out = c_out;
  d.groups = groups;
  d.in[0] = l_in;
  d.out[0] = l_out;
  d.k[0] = k;
  d.stride[0] = stride;
  d.pad[0] = padding;
  d.dilation[0] = dilation;
  d.a = a;
  d.b = b;
  d.bias = bias;
  return d;
}

bg_conv_desc desc2d(int op, bg_handle a, bg_handle b, bg_handle bias, int64_t n, int64_t c_in, int64_t h,
                    int64_t w, int64_t c_out, int64_t kh, int64_t kw, int64_t sh, int64_t sw, int64_t ph, int64_t pw,
                    int64_t dh, int64_t dw, int64_t groups, int64_t oh, int64_t ow) {
  bg_conv_desc d{};
  d.op = op;
  d.spatial = 2;
  d.n = n;
  d.c_in = c_in;
  d.c_out = c_out;
  d.groups = groups;
  d.in[0] = h;
  d.in[1] = w;
  d.out[0] = oh;
  d.out[1] = ow;
  d.k[0] = kh;
  d.k[1] = kw;
  d.stride[0] = sh;
  d.stride[1] = sw;
  d.pad[0] = ph;
  d.pad[1] = pw;
  d.dilation[0] = dh;
  d.dilation[1] = dw;
  d.a = a;
  d.b = b;
  d.bias = bias;
  return d;
}

}  // namespace

extern "C" {

int bg_conv_ex(bg_ctx* ctx, const bg_conv_desc* desc, bg_handle* out) {
  BG_API_BEGIN
  if (!desc || !out) fail(BG_E_INVALID, "HIP bridge: conv_ex desc and out must be non-NULL");
  *out = run_conv(ctx, *desc);
  BG_API_END
}

int bg_conv1d(bg_ctx* ctx, bg_handle input, bg_handle weight, bg_handle bias, int64_t n, int64_t c_in, int64_t l_in,
              int64_t c_out, int64_t k, int64_t stride, int64_t padding, int64_t dilation, int64_t groups,
              int64_t l_out, int dtype, bg_handle* out) {
  BG_API_BEGIN
  need_f32(dtype, "conv1d");
  *out = run_conv(ctx, desc1d(BG_CONV_FORWARD, input, weight, bias, n, c_in, l_in, c_out, k, stride, padding,
                              dilation, groups, l_out));
  BG_API_END
}

int bg_conv1d_backward_input(bg_ctx* ctx, bg_handle dy, bg_handle weight, int64_t n, int64_t c_in, int64_t l_in,
                             int64_t c_out, int64_t k, int64_t stride, int64_t padding, int64_t dilation,
                             int64_t groups, int64_t l_out, int dtype, bg_handle* out) {
  BG_API_BEGIN
  need_f32(dtype, "conv1d_backward_input");
  *out = run_conv(ctx, desc1d(BG_CONV_BACKWARD_INPUT, dy, weight, 0, n, c_in, l_in, c_out, k, stride, padding,
                              dilation, groups, l_out));
  BG_API_END
}

int bg_conv1d_backward_weight(bg_ctx* ctx, bg_handle dy, bg_handle input, int64_t n, int64_t c_in, int64_t l_in,
                              int64_t c_out, int64_t k, int64_t stride, int64_t padding, int64_t dilation,
                              int64_t groups, int64_t l_out, int dtype, bg_handle* out) {
  BG_API_BEGIN
  need_f32(dtype, "conv1d_backward_weight");
  *out = run_conv(ctx, desc1d(BG_CONV_BACKWARD_WEIGHT, dy, input, 0, n, c_in, l_in, c_out, k, stride, padding,
                              dilation, groups, l_out));
  BG_API_END
}

int bg_conv1d_backward_bias(bg_ctx* ctx, bg_handle dy, int64_t n, int64_t c_out, int64_t l_out, int dtype,
                            bg_handle* out) {
  BG_API_BEGIN
  need_f32(dtype, "conv1d_backward_bias");
  // realizer.ts:1270-1276: only n, cOut and lOut are validated.
  *out = run_conv(ctx, desc1d(BG_CONV_BACKWARD_BIAS, dy, 0, 0, n, c_out, l_out, c_out, 1, 1, 0, 1, 1, l_out));
  BG_API_END
}

int bg_conv2d(bg_ctx* ctx, bg_handle input, bg_handle weight, bg_handle bias, int64_t n, int64_t c_in, int64_t h,
              int64_t w, int64_t c_out, int64_t kh, int64_t kw, int64_t stride_h, int64_t stride_w, int64_t pad_h,
              int64_t pad_w, int64_t dilation_h, int64_t dilation_w, int64_t groups, int64_t out_h, int64_t out_w,
              int dtype, bg_handle* out) {
  BG_API_BEGIN
  need_f32(dtype, "conv2d");
  *out = run_conv(ctx, desc2d(BG_CONV_FORWARD, input, weight, bias, n, c_in, h, w, c_out, kh, kw, stride_h, stride_w,
                              pad_h, pad_w, dilation_h, dilation_w, groups, out_h, out_w));
  BG_API_END
}

int bg_conv2d_backward_input(bg_ctx* ctx, bg_handle dy, bg_handle weight, int64_t n, int64_t c_in, int64_t h,
                             int64_t w, int64_t c_out, int64_t kh, int64_t kw, int64_t stride_h, int64_t stride_w,
                             int64_t pad_h, int64_t pad_w, int64_t dilation_h, int64_t dilation_w, int64_t groups,
                             int64_t out_h, int64_t out_w, int dtype, bg_handle* out) {
  BG_API_BEGIN
  need_f32(dtype, "conv2d_backward_input");
  *out = run_conv(ctx, desc2d(BG_CONV_BACKWARD_INPUT, dy, weight, 0, n, c_in, h, w, c_out, kh, kw, stride_h,
                              stride_w, pad_h, pad_w, dilation_h, dilation_w, groups, out_h, out_w));
  BG_API_END
}

int bg_conv2d_backward_weight(bg_ctx* ctx, bg_handle dy, bg_handle input, int64_t n, int64_t c_in, int64_t h,
                              int64_t w, int64_t c_out, int64_t kh, int64_t kw, int64_t stride_h, int64_t stride_w,
                              int64_t pad_h, int64_t pad_w, int64_t dilation_h, int64_t dilation_w, int64_t groups,
                              int64_t out_h, int64_t out_w, int dtype, bg_handle* out) {
  BG_API_BEGIN
  need_f32(dtype, "conv2d_backward_weight");
  *out = run_conv(ctx, desc2d(BG_CONV_BACKWARD_WEIGHT, dy, input, 0, n, c_in, h, w, c_out, kh, kw, stride_h,
                              stride_w, pad_h, pad_w, dilation_h, dilation_w, groups, out_h, out_w));
  BG_API_END
}

int bg_conv2d_backward_bias(bg_ctx* ctx, bg_handle dy, int64_t n, int64_t c_out, int64_t out_h, int64_t out_w,
                            int dtype, bg_handle* out) {
  BG_API_BEGIN
  need_f32(dtype, "conv2d_backward_bias");
  *out = run_conv(ctx, desc2d(BG_CONV_BACKWARD_BIAS, dy, 0, 0, n, c_out, out_h, out_w, c_out, 1, 1, 1, 1, 0, 0, 1, 1,
                              1, out_h, out_w));
  BG_API_END
}

}  // extern "C"

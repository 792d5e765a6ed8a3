// Host-side tables the prologue and the plan take as inputs: RoPE pair
// tables, token positions and landmark frames. Pure C++, no device code.
#include <cmath>
#include <cstdint>
#include <vector>

#include "../../include/ch3hip.h"

extern "C" {

int h3hip_rope_pairs_axes(double theta, int32_t dim_t, int32_t dim_h, int32_t dim_w,
                          int32_t* pair_axis, float* pair_inv_freq) {
  if (!pair_axis || !pair_inv_freq || theta <= 0.0 || dim_t < 0 || dim_h < 0 || dim_w < 0 ||
      dim_t % 2 || dim_h % 2 || dim_w % 2)
    return H3HIP_EINVAL;
  const int32_t dims[3] = {dim_t, dim_h, dim_w};
  int32_t n = 0;
  for (int32_t axis = 0; axis < 3; axis++) {
    const double dim = static_cast<double>(dims[axis]);
    for (int32_t i = 0; i < dims[axis] / 2; i++) {
      pair_axis[n] = axis;
      pair_inv_freq[n] = static_cast<float>(1.0 / std::pow(theta, (2.0 * i) / dim));
      n++;
    }
  }
  return n;
}

int h3hip_rope_pairs_h3(const float* inv_freq, int32_t n_freq, int32_t* pair_axis,
                        float* pair_inv_freq) {
  if (!inv_freq || !pair_axis || !pair_inv_freq || n_freq <= 0) return H3HIP_EINVAL;
  // angles = cat(pos_t * f, pos_h * f, pos_w * f) (H3Transformer.swift:64-70).
  for (int32_t axis = 0; axis < 3; axis++)
    for (int32_t i = 0; i < n_freq; i++) {
      pair_axis[axis * n_freq + i] = axis;
      pair_inv_freq[axis * n_freq + i] = inv_freq[i];
    }
  return 3 * n_freq;
}

int h3hip_positions_grid(int32_t prefix_len, int32_t frames, int32_t height, int32_t width,
                         float* pos) {
  if (!pos || prefix_len < 0 || frames < 0 || height < 0 || width < 0) return H3HIP_EINVAL;
  float* p = pos;
  for (int32_t i = 0; i < prefix_len; i++, p += 3) p[0] = p[1] = p[2] = 0.f;
  for (int32_t t = 0; t < frames; t++)
    for (int32_t y = 0; y < height; y++)
      for (int32_t x = 0; x < width; x++, p += 3) {
        p[0] = static_cast<float>(t);
        p[1] = static_cast<float>(y);
        p[2] = static_cast<float>(x);
      }
  return prefix_len + frames * height * width;
}

int h3hip_positions_packed(int32_t text_tokens, int32_t audio_t, int32_t latent_t,
                           int32_t latent_h, int32_t latent_w, int32_t patch, double* pos) {
  if (!pos || text_tokens < 0 || audio_t < 0 || latent_t < 0 || patch <= 0) return H3HIP_EINVAL;
  // PositionGrid.axis (PackedSequence.swift:66-76): area-normalised linspace.
  const double area = std::sqrt(static_cast<double>(latent_h) * static_cast<double>(latent_w));
  auto axis = [&](int32_t dim, std::vector<double>& out) {
    const double ratio = static_cast<double>(dim) / area;
    const int32_t n = dim / patch;
    if (n <= 0) return false;
    const double step = ratio / static_cast<double>(n);
    const double origin = (1.0 - ratio) / 2.0;
    out.resize(n);
    for (int32_t i = 0; i < n; i++) out[i] = (static_cast<double>(i) * step + origin) * 32.0;
    return true;
  };
  std::vector<double> h_axis, w_axis;
  if (!axis(latent_h, h_axis) || !axis(latent_w, w_axis)) return H3HIP_EINVAL;
  double* p = pos;
  for (int32_t i = 0; i < text_tokens; i++, p += 3) {
    p[0] = static_cast<double>(i);
    p[1] = 0.0;
    p[2] = 0.0;
  }
  const double cursor = static_cast<double>(text_tokens);
  // Target audio: two rows per audio step, pinned to the w axis extremes.
  for (const double w : {w_axis.front(), w_axis.back()})
    for (int32_t i = 0; i < audio_t; i++, p += 3) {
      p[0] = cursor + static_cast<double>(i);
      p[1] = 0.0;
      p[2] = w;
    }
  // Target video: videoTGrid origin + exclusive cumsum of 5/3 * [1,4,4,4,4].
  static const int kFramesPerToken[5] = {1, 4, 4, 4, 4};
  const double rescale = 5.0 / 3.0;
  double t = cursor;
  for (int32_t f = 0; f < latent_t; f++) {
    for (const double hv : h_axis)
      for (const double wv : w_axis) {
        p[0] = t;
        p[1] = hv;
        p[2] = wv;
        p += 3;
      }
    t += rescale * static_cast<double>(kFramesPerToken[f % 5]);
  }
  return static_cast<int>((p - pos) / 3);
}

int h3hip_landmarks(int32_t frames, int32_t n, int32_t* out) {
  if (!out || frames <= 0) return H3HIP_EINVAL;
  int32_t count = n < 2 ? 2 : n;
  if (count >= frames) {
    for (int32_t i = 0; i < frames; i++) out[i] = i;
    return frames;
  }
  int32_t written = 0;
  for (int32_t i = 0; i < count; i++) {
    // Swift's .rounded() rounds half away from zero, as std::round does.
    const int32_t f = static_cast<int32_t>(
        std::round(static_cast<double>(i) * static_cast<double>(frames - 1) /
                   static_cast<double>(count - 1)));
    if (written == 0 || out[written - 1] != f) out[written++] = f;
  }
  return written;
}

}  // extern "C"

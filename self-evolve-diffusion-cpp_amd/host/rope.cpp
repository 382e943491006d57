// RoPE (cos, sin) tables — see sd/rope.h.
#include "sd/rope.h"

#include <algorithm>
#include <cmath>
#include <stdexcept>

namespace sd {

namespace {

// Split of a head's complex pairs over the t, h, w axes (blocks.h:39-44):
// t_real = d - 4*(d/6) real dims for t, s_real = 2*(d/6) for h and for w;
// the frequency of pair j on an axis of `real` dims is theta^(-2j/real),
// evaluated in float as the reference does (std::pow on floats).
int t_real_dims(int d) { return d - 4 * (d / 6); }
int s_real_dims(int d) { return 2 * (d / 6); }

std::vector<float> axis_freqs(int pairs, int real, float theta) {
  std::vector<float> f((size_t)pairs);
  for (int j = 0; j < pairs; j++) f[(size_t)j] = std::pow(theta, -2.f * (float)j / (float)real);
  return f;
}

void put(float* cs, float ang) {
  cs[0] = std::cos(ang);
  cs[1] = std::sin(ang);
}

}  // namespace

// blocks.cpp:46-67: angle of pair j = t*ft[j] (j < ct), h*fs[j-ct], w*fs[j-ct-cs].
RopeTable rope_table_3d(int T, int H, int W, int d, float theta) {
  if (T < 0 || H < 0 || W < 0 || d <= 0 || d % 2)
    throw std::invalid_argument("rope_table_3d: bad grid or head_dim");
  const int ct = t_real_dims(d) / 2, cs = s_real_dims(d) / 2;
  const std::vector<float> ft = axis_freqs(ct, t_real_dims(d), theta);
  const std::vector<float> fs = axis_freqs(cs, s_real_dims(d), theta);
  RopeTable r;
  r.n_rot = ct + 2 * cs;
  r.L = (int64_t)T * H * W;
  r.cs.resize((size_t)r.L * r.n_rot * 2);
  float* p = r.cs.data();
  for (int t = 0; t < T; t++)
    for (int h = 0; h < H; h++)
      for (int w = 0; w < W; w++)
        for (int j = 0; j < r.n_rot; j++, p += 2) {
          float ang;
          if (j < ct)
            ang = (float)t * ft[(size_t)j];
          else if (j < ct + cs)
            ang = (float)h * fs[(size_t)(j - ct)];
          else
            ang = (float)w * fs[(size_t)(j - ct - cs)];
          put(p, ang);
        }
  return r;
}

// blocks.cpp:69-84: angle = fl(fl(l * scaling) * theta^(-2j/t_real)), j < t_real/2.
RopeTable rope_table_1d(int L, int d, float theta, float scaling) {
  if (L < 0 || d <= 0 || d % 2) throw std::invalid_argument("rope_table_1d: bad length or head_dim");
  RopeTable r;
  r.n_rot = t_real_dims(d) / 2;
  r.L = L;
  const std::vector<float> f = axis_freqs(r.n_rot, t_real_dims(d), theta);
  r.cs.resize((size_t)L * r.n_rot * 2);
  float* p = r.cs.data();
  for (int l = 0; l < L; l++)
    for (int j = 0; j < r.n_rot; j++, p += 2) put(p, (float)l * scaling * f[(size_t)j]);
  return r;
}

}  // namespace sd

extern "C" {

int sd_rope_table_3d(int T, int H, int W, int head_dim, float theta, float* cs) {
  try {
    if (!cs) {
      if (head_dim <= 0 || head_dim % 2) return -1;
      return (head_dim - 4 * (head_dim / 6)) / 2 + 2 * (head_dim / 6);
    }
    sd::RopeTable r = sd::rope_table_3d(T, H, W, head_dim, theta);
    std::copy(r.cs.begin(), r.cs.end(), cs);
    return r.n_rot;
  } catch (const std::exception&) {
    return -1;
  }
}

int sd_rope_table_1d(int L, int head_dim, float theta, float scaling, float* cs) {
  try {
    if (!cs) {
      if (head_dim <= 0 || head_dim % 2) return -1;
      return (head_dim - 4 * (head_dim / 6)) / 2;
    }
    sd::RopeTable r = sd::rope_table_1d(L, head_dim, theta, scaling);
    std::copy(r.cs.begin(), r.cs.end(), cs);
    return r.n_rot;
  } catch (const std::exception&) {
    return -1;
  }
}

}  // extern "C"

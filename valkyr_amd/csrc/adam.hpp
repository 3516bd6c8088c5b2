// The Adam update of one element (adam_step.comp:41-62), shared by every
// kernel that applies it (the streaming spans, the norm-gain spans, the
// embedding rows) so that all of them round identically.
#pragma once

#include "common.hpp"

namespace vkh {

struct AdamHyper {
    float lr, b1, b2, eps, bc1, bc2, wd;  // bc1 = 1 - beta1^t, bc2 = 1 - beta2^t
};

VKH_DEV void adam1(float &p, float g, float &m, float &v, float lr, float b1, float b2, float eps,
                   float bc1, float bc2, float wd) {
#pragma clang fp contract(off)
    const float nm = b1 * m + (1.0f - b1) * g;
    const float nv = b2 * v + (1.0f - b2) * g * g;
    m = nm;
    v = nv;
    const float m_hat = nm / bc1;
    const float v_hat = nv / bc2;
    float q = p;
    if (wd > 0.0f) q = q * (1.0f - lr * wd);
    p = q - lr * m_hat / (sqrtf(v_hat) + eps);
}

VKH_DEV void adam4(f32x4 &p, const f32x4 &g, f32x4 &m, f32x4 &v, float lr, float b1, float b2,
                   float eps, float bc1, float bc2, float wd) {
    float pp[4] = {p.x, p.y, p.z, p.w}, mm[4] = {m.x, m.y, m.z, m.w}, vv[4] = {v.x, v.y, v.z, v.w};
    const float gg[4] = {g.x, g.y, g.z, g.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) adam1(pp[i], gg[i], mm[i], vv[i], lr, b1, b2, eps, bc1, bc2, wd);
    p = f32x4{pp[0], pp[1], pp[2], pp[3]};
    m = f32x4{mm[0], mm[1], mm[2], mm[3]};
    v = f32x4{vv[0], vv[1], vv[2], vv[3]};
}

VKH_DEV void adam4(f32x4 &p, const f32x4 &g, f32x4 &m, f32x4 &v, const AdamHyper &h) {
    adam4(p, g, m, v, h.lr, h.b1, h.b2, h.eps, h.bc1, h.bc2, h.wd);
}

}  // namespace vkh

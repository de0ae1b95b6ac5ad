// Host-side restatement of the joint-sequence layout and 3-axis RoPE tables
// the block consumes (integer bookkeeping plus one f32 table per step).
#include <math.h>
#include <string.h>

#include <vector>

#include "qimm.h"

namespace {
constexpr int64_t kTokensPerSlot = 4;     // src/joint_layout.rs:10
constexpr int64_t kRopeNeg = 1024;        // src/rope.rs:41-47
constexpr int64_t kRopePos = 8192;
}  // namespace

extern "C" {

// JointLayout::new, src/joint_layout.rs:52-103.
int qimm_joint_layout(int64_t text_len, const uint8_t *text_image_mask, const int64_t *cond_shapes,
                      int64_t ncond, int64_t target_h, int64_t target_w, int64_t *image_ids, int64_t cap,
                      int64_t *prefix_len, int64_t *target_len, int64_t *total_len) {
    if (text_len < 0 || ncond < 0 || target_h < 0 || target_w < 0 || !prefix_len || !target_len ||
        !total_len || (ncond > 0 && !cond_shapes) || (cap > 0 && !image_ids))
        return QIMM_ERR_ARG;
    std::vector<int64_t> ids;
    int64_t i = 0, next_image = 0;
    auto slot = [&](int64_t j) { return text_image_mask && text_image_mask[j] != 0; };
    while (i < text_len) {
        if (!slot(i)) {
            while (i < text_len && !slot(i)) {
                ids.push_back(-1);
                i++;
            }
            continue;
        }
        // condition blocks are delimited by token counts, not by slot runs
        if (next_image >= ncond) return QIMM_ERR_SHAPE;  // more image slots than images
        const int64_t h = cond_shapes[2 * next_image], w = cond_shapes[2 * next_image + 1];
        const int64_t needed = h * w / kTokensPerSlot;
        int64_t have = 0;
        for (int64_t j = i; j < text_len && j < i + needed; j++) have += slot(j);
        if ((h * w) % kTokensPerSlot || have != needed) return QIMM_ERR_SHAPE;
        ids.insert(ids.end(), (size_t)(h * w), next_image);
        next_image++;
        i += needed;
    }
    if (next_image != ncond) return QIMM_ERR_SHAPE;  // images without slots
    ids.insert(ids.end(), (size_t)(target_h * target_w), ncond);
    *target_len = target_h * target_w;
    *total_len = (int64_t)ids.size();
    *prefix_len = *total_len - *target_len;
    if (cap < *total_len) return QIMM_ERR_ARG;
    if (!ids.empty()) memcpy(image_ids, ids.data(), ids.size() * sizeof(int64_t));
    return QIMM_OK;
}

// EmbedNd::forward (src/rope.rs:104-211) over the tables of
// EmbedNd::new_with_mode (src/rope.rs:37-88): per axis, f32
// inv_freq_i = exp(i * f32(-2 ln(theta) / dim)), angle = position * inv_freq,
// (cos, sin) gathered at position + 1024.
int qimm_rope_table(const int64_t *shapes, int64_t nshapes, const uint8_t *image_mask, int64_t seq,
                    const int64_t axes[3], double theta, float *pe) {
    if (seq < 0 || nshapes < 0 || (nshapes && !shapes) || (seq && (!image_mask || !pe)) || !axes)
        return QIMM_ERR_ARG;
    for (int a = 0; a < 3; a++)
        if (axes[a] <= 0 || axes[a] % 2) return QIMM_ERR_SHAPE;
    std::vector<int64_t> pos[3];
    int64_t cursor = 0, position = 0;
    auto text_token = [&]() {
        for (int a = 0; a < 3; a++) pos[a].push_back(position);
        position++;
    };
    for (int64_t b = 0; b < nshapes; b++) {
        const int64_t frame = shapes[3 * b], height = shapes[3 * b + 1], width = shapes[3 * b + 2];
        const int64_t block_tokens = frame * height * width;
        int64_t start = seq;
        for (int64_t t = cursor; t < seq; t++)
            if (image_mask[t]) {
                start = t;
                break;
            }
        for (int64_t t = cursor; t < start; t++) text_token();
        cursor = start;
        pos[0].insert(pos[0].end(), (size_t)block_tokens, position);  // frame frozen
        position += height > width ? height : width;
        const int64_t h0 = -(height - height / 2), w0 = -(width - width / 2);
        for (int64_t h = 0; h < height; h++)
            for (int64_t w = 0; w < width; w++) {
                pos[1].push_back(h0 + h);
                pos[2].push_back(w0 + w);
            }
        cursor += block_tokens;
    }
    for (int64_t t = cursor; t < seq; t++) text_token();
    for (int a = 0; a < 3; a++)
        if ((int64_t)pos[a].size() != seq) return QIMM_ERR_SHAPE;
    const int64_t width_total = axes[0] + axes[1] + axes[2];
    const double ln_theta = log((double)(float)theta);
    for (int a = 0; a < 3; a++) {
        const float mul = (float)(-2.0 * ln_theta / (double)axes[a]);
        int64_t col0 = 0;
        for (int b = 0; b < a; b++) col0 += axes[b] / 2;
        for (int64_t t = 0; t < seq; t++) {
            const int64_t p = pos[a][t];
            if (p < -kRopeNeg || p >= kRopePos) return QIMM_ERR_SHAPE;
            float *row = pe + t * width_total;
            for (int64_t i = 0; i < axes[a] / 2; i++) {
                const float inv_freq = expf((float)i * mul);
                const float ang = (float)p * inv_freq;
                row[2 * (col0 + i)] = cosf(ang);
                row[2 * (col0 + i) + 1] = sinf(ang);
            }
        }
    }
    return QIMM_OK;
}

}  // extern "C"

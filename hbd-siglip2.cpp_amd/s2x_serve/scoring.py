"""Embedding normalization and SigLIP2's sigmoid image-text scores (host,
numpy; no GPU).

    l2_normalize:  x * f32(1 / (sqrt(sum x^2) + 1e-12)), the sum in double
                   (src/siglip2_server.cpp:126-131)
    score:         logit[i, j] = f32(dot(img_n[i], txt_n[j]) * exp(logit_scale)
                   + logit_bias), dot in double over the normalized rows;
                   prob = sigmoid(logit) in the overflow-free split form
                   (src/siglip2_score.cpp:77-134)
"""
import numpy as np


def l2_normalize(v):
    """Each row of v (float32) scaled to unit length."""
    v = np.array(v, np.float32, ndmin=2)
    s = np.sum(v.astype(np.float64) ** 2, axis=1, keepdims=True)
    inv = (1.0 / (np.sqrt(s) + 1e-12)).astype(np.float32)
    return v * inv


def sigmoid(x):
    x = np.asarray(x, np.float32)
    out = np.empty_like(x)
    pos = x >= 0
    e = np.exp(-x[pos])
    out[pos] = np.float32(1.0) / (np.float32(1.0) + e)
    e = np.exp(x[~pos])
    out[~pos] = e / (np.float32(1.0) + e)
    return out


def score_image_text(image_embeds, text_embeds, logit_scale, logit_bias):
    """(logits, probs), both (n_image, n_text) float32."""
    img = l2_normalize(image_embeds).astype(np.float64)
    txt = l2_normalize(text_embeds).astype(np.float64)
    scale = float(np.exp(np.float32(logit_scale)))
    logits = (img @ txt.T * scale + float(np.float32(logit_bias))).astype(np.float32)
    return logits, sigmoid(logits)

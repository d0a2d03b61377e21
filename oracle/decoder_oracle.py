"""CPU oracle of the llama2c decoder (loom-private/llama2c-decoder) in numpy.

TEST INFRASTRUCTURE ONLY: imported by tests/ as the checker of the decoder's
kernels and application. The product never imports it.

Restates, from the reference repository:
  model            contract.json "data_generation" (decoder.cu:27-43)
  prompts          oracle.cpp:76-78
  analytic_tokens  oracle.cpp:83-92 (token after step s: (prompt + s + 1) mod vocab)
  probe_sequences  oracle.cpp:94-100
  dense_double     oracle.cpp:30-72 (every classifier row against every column, in double)
  invariants       oracle.cpp:128-162 (mean square and probability sum within upstream's bounds)
  within           oracle.cpp:74-78, tolerances contract.json "tolerances"

How it is pinned (tests/test_decoder.py):
  * analytic_tokens reproduces the expected token lists that contract.json
    records for upstream's smoke and validation configurations;
  * dense_double equals the closed forms of the synthetic model
    (scale = 1 / sqrt((width + 15) / width + 1e-5); one normalized entry 4 scale,
    the rest scale; logits the same values rotated; probabilities e^{3 scale} / Z
    and 1 / Z) and its argmax reproduces analytic_tokens;
  * a planted mistake (the classifier's offset changed) breaks that agreement.
"""
from __future__ import annotations

import numpy as np

# contract.json "tolerances" / oracle.cpp:23-27.
NORMALIZED_RELATIVE = 2.0e-6
LOGIT_RELATIVE = 2.0e-6
PROBABILITY_RELATIVE = 2.0e-5
ABSOLUTE_FLOOR = 1.0e-12


def model(width: int, vocab: int, classifier_offset: int = -1):
    """(embedding, classifier, norm_weight) as float32: embedding[t][j] = 4 if
    j == t else 1; classifier[r][j] = 1 if j == (r + offset) mod vocab else 0
    (offset -1 is the contract's); norm weight 1."""
    embedding = np.ones((vocab, width), np.float32)
    embedding[np.arange(vocab), np.arange(vocab)] = 4.0
    classifier = np.zeros((vocab, width), np.float32)
    classifier[np.arange(vocab), (np.arange(vocab) + classifier_offset) % vocab] = 1.0
    return embedding, classifier, np.ones(width, np.float32)


def prompts(batch: int, vocab: int) -> np.ndarray:
    return (np.arange(batch) % vocab).astype(np.int32)


def analytic_tokens(batch: int, vocab: int, steps: int, first_prompt: int = 0) -> np.ndarray:
    """[batch][steps] int32: the token each step produces."""
    start = (np.arange(batch) + first_prompt) % vocab
    return ((start[:, None] + np.arange(1, steps + 1)[None, :]) % vocab).astype(np.int32)


def probe_sequences(batch: int) -> list[int]:
    count = min(8, batch)
    out: list[int] = []
    for i in range(count):
        b = 0 if count == 1 else i * (batch - 1) // (count - 1)
        if not out or out[-1] != b:
            out.append(b)
    return out


def dense_double(prompt: int, width: int, vocab: int, steps: int, classifier_offset: int = -1):
    """Every step of one sequence in double: (normalized [steps][width],
    logits [steps][vocab], probabilities [steps][vocab], tokens [steps])."""
    embedding, classifier, weight = model(width, vocab, classifier_offset)
    E, C, w = embedding.astype(np.float64), classifier.astype(np.float64), weight.astype(np.float64)
    token = prompt % vocab
    normalized = np.empty((steps, width))
    logits = np.empty((steps, vocab))
    probabilities = np.empty((steps, vocab))
    tokens = np.empty(steps, np.int64)
    for s in range(steps):
        x = E[token]
        scale = 1.0 / np.sqrt(np.sum(x * x) / width + 1.0e-5)
        o = w * (scale * x)
        l = C @ o  # dense: every row against every column
        p = np.exp(l - l.max())
        p /= p.sum()
        token = int(np.argmax(p))  # first maximum
        normalized[s], logits[s], probabilities[s], tokens[s] = o, l, p, token
    return normalized, logits, probabilities, tokens


def closed_form(prompt: int, width: int, vocab: int, steps: int):
    """The synthetic model's values in closed form (double), as dense_double
    returns them."""
    scale = 1.0 / np.sqrt((width + 15.0) / width + 1.0e-5)
    normalized = np.full((steps, width), scale)
    logits = np.full((steps, vocab), scale)
    top = np.exp(3.0 * scale)
    z = top + (vocab - 1)
    probabilities = np.full((steps, vocab), 1.0 / z)
    tokens = np.empty(steps, np.int64)
    token = prompt % vocab
    for s in range(steps):
        normalized[s, token] = 4.0 * scale
        nxt = (token + 1) % vocab
        logits[s, nxt] = 4.0 * scale
        probabilities[s, nxt] = top / z
        tokens[s] = nxt
        token = nxt
    return normalized, logits, probabilities, tokens


def within(observed, expected, relative) -> np.ndarray:
    observed = np.asarray(observed, np.float64)
    expected = np.asarray(expected, np.float64)
    return np.abs(observed - expected) <= relative * np.abs(expected) + ABSOLUTE_FLOOR


def invariants(normalized: np.ndarray, probabilities: np.ndarray, width: int, vocab: int):
    """Upstream's normalization invariants for rows of float32 outputs:
    (mean-square ok, probability-sum ok) boolean arrays."""
    square_bound = np.float32(2.0e-5) + np.float32(1.2e-7) * np.float32(width)
    sum_bound = np.float32(1.0e-6) + np.float32(1.2e-7) * np.float32(vocab)
    o = normalized.reshape(-1, width).astype(np.float64)
    p = probabilities.reshape(-1, vocab).astype(np.float64)
    mean_square = (np.sum(o * o, axis=1) / width).astype(np.float32)
    psum = np.sum(p, axis=1).astype(np.float32)
    return (np.abs(mean_square - np.float32(1)) <= square_bound,
            np.abs(psum - np.float32(1)) <= sum_bound)


def rmsnorm_f32(x: np.ndarray, weight: np.ndarray) -> np.ndarray:
    """The float32 operation order of the contract's rmsnorm for rows x whose
    square sum is exact in float32 (true for the synthetic model): ss / width,
    + 1e-5f, 1 / sqrtf, then w * (scale * x), each step rounded to float32."""
    x = x.astype(np.float32)
    ss = np.sum(x.astype(np.float64) ** 2, axis=-1)
    assert np.all(ss < 2.0 ** 24), "square sum must be exact in float32"
    ss = ss.astype(np.float32)
    ss = ss / np.float32(x.shape[-1])
    ss = ss + np.float32(1e-5)
    scale = np.float32(1.0) / np.sqrt(ss)
    return weight.astype(np.float32) * (scale[..., None] * x)

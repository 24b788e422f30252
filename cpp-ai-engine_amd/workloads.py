"""Seeded synthetic workloads of the training path: inputs and initial parameters.

Every generator is a pure function of its seed (numpy's PCG64 through default_rng), so the
benchmark, the GPU parity tests and the golden-fixture scripts that feed the compiled
reference all see the same bits.

Parameter vectors are flat float32 in the engine's parameter order, which is the
reference's Module::parameters() order:
  - the character model of examples/charlm_demo.cpp:57-87 is the embedding table, then per
    block (src/transformer.cpp:416-425) norm1 (gamma, beta), norm2 (gamma, beta), the query,
    key, value and output projections (weight (in, out), bias (1, out) each,
    src/transformer.cpp:360-367), ff1 and ff2; then the head (weight, bias);
  - initial values follow the reference's own initialisers: Linear weights Xavier-uniform
    with limit sqrt(6 / (in + out)) and zero biases (src/nn.cpp:85-99), the embedding
    N(0, 0.02) (src/transformer.cpp:203), LayerNorm gamma 1 and beta 0
    (src/transformer.cpp:18-31). The values are drawn here rather than by the reference's
    mt19937, so both engines can be handed the same vector.
"""
import numpy as np

# (batch, seq, vocab, d_model, heads, ffn, layers): BASELINE configs 3 and 5.
CHARLM_CFG3 = (32, 64, 121, 96, 4, 384, 2)
TRANSFORMER_CFG5 = (16, 512, 256, 1024, 16, 4096, 12)


def cnn_inputs(seed=2, batch=64):
    """cfg 2: pixels U[0,1] (batch, 1, 28, 28), labels U{0..9}, Kaiming-uniform conv and
    Linear weights (limit sqrt(6 / fan_in)), zero biases."""
    r = np.random.default_rng(seed)
    x = r.uniform(0.0, 1.0, (batch, 1, 28, 28)).astype(np.float32)
    labels = r.integers(0, 10, batch)
    shapes = [(8, 1, 3, 3), (8,), (16, 8, 3, 3), (16,), (784, 10), (1, 10)]
    params = []
    for shp in shapes:
        n = int(np.prod(shp))
        if len(shp) == 1 or shp[0] == 1:
            params.append(np.zeros(n, np.float32))
        else:
            fan_in = int(np.prod(shp[1:])) if len(shp) == 4 else shp[0]
            lim = np.sqrt(6.0 / fan_in)
            params.append(r.uniform(-lim, lim, n).astype(np.float32))
    return x, labels, np.concatenate(params)


def lm_inputs(seed, batch, seq, vocab):
    """Token ids U{0..vocab-1} as float32 (batch, seq), as Embedding expects them, and next
    tokens U{0..vocab-1} (batch * seq) as int64 class labels."""
    r = np.random.default_rng(seed)
    ids = r.integers(0, vocab, (batch, seq)).astype(np.float32)
    targets = r.integers(0, vocab, batch * seq)
    return ids, targets


def lm_param_layout(vocab, d, ff, layers):
    """[(name, shape, kind)] of the character model in parameter order; kind is one of
    'embedding', 'gamma', 'beta', 'weight', 'bias'."""
    out = [("embedding.weight", (vocab, d), "embedding")]
    for i in range(layers):
        p = f"block{i}."
        for norm in ("norm1", "norm2"):
            out += [(p + norm + ".gamma", (d,), "gamma"), (p + norm + ".beta", (d,), "beta")]
        for proj in ("query", "key", "value", "out"):
            out += [(p + "attn." + proj + ".weight", (d, d), "weight"),
                    (p + "attn." + proj + ".bias", (1, d), "bias")]
        out += [(p + "ff1.weight", (d, ff), "weight"), (p + "ff1.bias", (1, ff), "bias"),
                (p + "ff2.weight", (ff, d), "weight"), (p + "ff2.bias", (1, d), "bias")]
    out += [("head.weight", (d, vocab), "weight"), ("head.bias", (1, vocab), "bias")]
    return out


def lm_param_offsets(vocab, d, ff, layers):
    """{name: (offset, shape)} into the flat parameter vector."""
    offs, off = {}, 0
    for name, shape, _ in lm_param_layout(vocab, d, ff, layers):
        offs[name] = (off, shape)
        off += int(np.prod(shape))
    return offs


def lm_init_params(seed, vocab, d, ff, layers):
    """The reference initialisers' distributions, drawn from one seed, flat float32."""
    r = np.random.default_rng(seed)
    parts = []
    for _, shape, kind in lm_param_layout(vocab, d, ff, layers):
        n = int(np.prod(shape))
        if kind == "embedding":
            parts.append((r.standard_normal(n, dtype=np.float32) * np.float32(0.02)))
        elif kind == "gamma":
            parts.append(np.ones(n, np.float32))
        elif kind in ("beta", "bias"):
            parts.append(np.zeros(n, np.float32))
        else:
            lim = np.float32(np.sqrt(6.0 / (shape[0] + shape[1])))
            parts.append(r.uniform(-lim, lim, n).astype(np.float32))
    return np.concatenate(parts)

"""The seeded whisper-large-v3-turbo weights with the decoder's token embedding (tied with the LM head)
scaled by 8 and every decoder projection (self- and cross-attention q/k/v/out, fc1, fc2) by 4. With the
N(0, 0.02) weights the greedy decoder of a random-init model falls into repeating one id (the seed-0
fixture's 224 ids hold 3 distinct ones); with these, the ids vary from step to step (62 distinct in
224). Powers of two, so the scaled fp16 values are exact. Shared by the fixture generator
(tests/golden/make_golden.py varied) and the GPU test that loads them as a local checkpoint.
"""

import numpy as np

EMBED_SCALE, PROJ_SCALE = 8.0, 4.0
FIXTURE_NAME = 'e2e_turbo_seed0_varied.json'


def is_scaled_projection(name):
    return (name.startswith('model.decoder.layers.') and name.endswith('.weight')
            and ('_proj.' in name or '.fc1.' in name or '.fc2.' in name))


def scaled_decoder(params):
    """A copy of the parameter dict (name -> fp16 numpy array) with the decoder scaled as above."""
    out = dict(params)
    for name, a in params.items():
        if name == 'model.decoder.embed_tokens.weight':
            out[name] = (a.astype(np.float32) * EMBED_SCALE).astype(np.float16)
        elif is_scaled_projection(name):
            out[name] = (a.astype(np.float32) * PROJ_SCALE).astype(np.float16)
    return out

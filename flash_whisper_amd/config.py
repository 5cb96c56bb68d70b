"""Model dimensions and the fixed synthetic decoding setup.

Dimensions are those of openai/whisper-large-v3-turbo (the model the reference benchmarks,
custom/model.py:40-47 reads them from its HF config). The prompt and suppress ids stand in for the
checkpoint's tokenizer and generation_config, which are not available offline: the reference takes
``PROMPT`` token strings through the tokenizer (custom/model.py:22,44) and the suppress lists from
``generation_config`` (custom/model.py:57-61). With random-init weights any fixed in-vocabulary ids
are equally valid, so they are fixed constants here.
"""

from dataclasses import dataclass, field

SAMPLE_RATE = 16000
N_SAMPLES = 30 * SAMPLE_RATE          # custom/model.py:21
N_FFT, HOP_LENGTH, N_MELS = 400, 160, 128
CHUNK = 8                             # decode steps per graph replay (custom/model.py:23)
SPLIT_KEYS = 64                       # keys per split block of the reference op (custom/selftest.py:13)

# <|startoftranscript|> <|en|> <|transcribe|> <|notimestamps|> in the v3 vocabulary (fixed, not looked up).
PROMPT_IDS = (50258, 50259, 50360, 50364)
EOS_IDS = (50257,)
# Fixed stand-ins for generation_config.suppress_tokens / begin_suppress_tokens.
SUPPRESS_IDS = (1, 2, 7, 8, 9, 10, 14, 25, 26, 27, 28, 29, 31, 58, 59, 60, 61, 62, 63, 90, 91, 92, 93,
                50254, 50258, 50359, 50360, 50361, 50362, 50363)
BEGIN_SUPPRESS_IDS = (220, 50257)


@dataclass(frozen=True)
class WhisperDims:
    n_mels: int = N_MELS
    d_model: int = 1280
    heads: int = 20
    ffn: int = 5120
    enc_layers: int = 32
    dec_layers: int = 4
    vocab: int = 51866
    enc_len: int = 1500            # max_source_positions
    max_pos: int = 448             # max_target_positions
    ln_eps: float = 1e-5

    @property
    def head_dim(self):
        return self.d_model // self.heads

    @property
    def mel_frames(self):
        return 2 * self.enc_len


TURBO = WhisperDims()


@dataclass(frozen=True)
class DecodeSetup:
    prompt: tuple = PROMPT_IDS
    eos: tuple = EOS_IDS
    suppress: tuple = SUPPRESS_IDS
    begin_suppress: tuple = BEGIN_SUPPRESS_IDS
    extra: dict = field(default_factory=dict)

"""Drop-in for custom/model.py: ``from custom.model import CustomModel`` (reference runner.py:153-156)."""

from flash_whisper_amd.config import CHUNK, N_SAMPLES, SAMPLE_RATE  # noqa: F401
from flash_whisper_amd.model import CustomModel  # noqa: F401

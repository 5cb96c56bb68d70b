"""MI355X-native (gfx950) batch-1 Whisper-large-v3-turbo hot path: HIP kernels behind a C ABI."""

__version__ = '0.1.0'

"""Drop-in entry points of sp4s-s/flash_whisper's `custom` package, backed by flash_whisper_amd."""

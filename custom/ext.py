"""Drop-in for custom/ext.py: ``load_ext()``; ``python -m custom.ext`` builds and prints resource usage."""

from flash_whisper_amd.build import BUILD_DIR  # noqa: F401
from flash_whisper_amd.ext import load_ext, main  # noqa: F401

if __name__ == '__main__':
    main()

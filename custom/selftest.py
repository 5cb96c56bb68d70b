"""Drop-in for custom/selftest.py: ``run_selftest(ext)``, ``workspace``, ``SPLIT_KEYS``; ``--out DIR``."""

from flash_whisper_amd.selftest import HEAD_DIM, HEADS, HIDDEN, SPLIT_KEYS, VOCAB, main, run_selftest, workspace  # noqa: F401

if __name__ == '__main__':
    main()

"""CPU oracle for the batch-1 Whisper hot path of sp4s-s/flash_whisper.

TEST INFRASTRUCTURE ONLY. This package restates the reference algorithm on the CPU (numpy) so the
HIP kernels can be checked against it. Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import it, and only to compare against or as the timed CPU baseline. The product
(``flash_whisper_amd``, ``custom``) never imports it and has no CPU fallback.

Modules and what pins each function (checks live in tests/test_oracle_*.py):
- ``logmel``: log-mel front end (custom/model.py:93-98; transformers feature_extraction_whisper.py:135-170).
  Pinned by the transformers mel filterbank and log-mel golden vectors (tests/golden/make_golden.py),
  Parseval/pure-tone closed forms and the Slaney mel-scale identities.
- ``decoder``: add_layernorm, split-free attention, LM head argmax, finalize and the decoder step
  (custom/kernels/whisper_kernels.cu:20-267, custom/model.py:107-123, custom/selftest.py:26-88).
  Pinned by a transformers WhisperForConditionalGeneration forward on a tiny random config (fp32),
  textbook LayerNorm/softmax identities and brute-force argmax on small inputs.
- ``encoder``: HF WhisperEncoder in fp16 semantics (transformers modeling_whisper.py:379-414, 592-648)
  and the cross K/V projection (custom/model.py:143-147). Pinned by the same transformers tiny-config
  golden vectors (fp32) and by conv1d/attention closed forms.
- ``torch_cpu``: the reference's PyTorch path (custom/pytorch_model.py:29-89: transformers Whisper, the
  feature extractor's torch log-mel, greedy loop over the HF KV cache) in fp32 on the host CPU, the
  timed CPU baseline of bench.py. Its loop is pinned by transformers' own greedy ids on a tiny model
  (tests/test_torch_cpu_baseline.py); it is a timing baseline, not the id check.
- ``pipeline``: waveform -> log-mel -> encoder -> cross K/V -> greedy ids (custom/model.py:173-225).
  Its parts are pinned as above; the fp16 rounding points themselves (which only matter at the ulp
  level) are the reference's, checked by construction against whisper_kernels.cu and HF's fp16 casts.
"""

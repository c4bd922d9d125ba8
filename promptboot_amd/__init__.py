"""MI355X (gfx950) decode-step token sampler for promptboot.

The product is the C ABI library libpbsample.so (include/pbsample.h) built
from promptboot_amd/csrc; promptboot_amd.sampler mirrors the reference's
sampler API over it, promptboot_amd.hip binds the HIP runtime for device
buffers, streams and events, promptboot_amd.wire and promptboot_amd.evidence
read and produce the reference's evidence formats, and
promptboot_amd.workloads builds seeded synthetic batches.
"""
from . import evidence, hip, sampler, wire, workloads  # noqa: F401
from .sampler import (  # noqa: F401
    BatchSampler, InferenceError, SamplingState, greedy_token, sample_token,
    sample_token_with_repetition, top_logits_8,
)

"""ferro_amd: MI355X (gfx950) token sampler for ferro - the penalty / top-k / top-p / softmax / draw / argmax /
draft-verification hot path as HIP kernels behind the C ABI of include/ferro_sampler.h."""
from .sampler import (PARAMS_DTYPE, Context, DeviceRng, Rng, Sampler, SamplerError, SamplerParams, argmax_batch,  # noqa: F401
                      decode_step, device_error, hist_append, lookup_draft, params_array, penalize_batch, sample_batch, verify)

"""klsample: MI355X-native (gfx950) fused token sampling.

Drop-in for the reference's ``serving/sampling.py`` (``SamplingParams``, ``Sampler``,
``SampleResult``) plus a batched entry point, running hand-written HIP kernels through
the C ABI of ``libklsample.so`` (``include/klsample.h``).
"""
from .sampling import SampleResult, Sampler, SamplingParams, sample_batch

__all__ = ['SamplingParams', 'SampleResult', 'Sampler', 'sample_batch']

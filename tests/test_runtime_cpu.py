"""Host-side runtime logic that needs no GPU (reference runtime.py:567-585)."""

from gdn_state_codec import GdnStateCodecRuntime


def test_decode_fallback_reasons():
    reason = GdnStateCodecRuntime.decode_fallback_reason
    assert reason(num_prefills=0, num_decodes=1, speculative=True) == "speculative decode"
    assert reason(num_prefills=1, num_decodes=1, speculative=False) == "mixed prefill/decode batch"
    assert reason(num_prefills=0, num_decodes=2, speculative=False) == "multi-request decode batch"
    assert (reason(num_prefills=0, num_decodes=1, speculative=False, cache_index_count=2)
            == "multi-request decode batch")
    assert reason(num_prefills=0, num_decodes=1, speculative=False, cache_index_count=1) is None
    assert reason(num_prefills=3, num_decodes=0, speculative=False) is None


def test_experiment_admits_the_reference_initializers():
    """Both initializers of the reference's configuration (config.py:62-86):
    quant_only with 0..32 power iterations, exact_svd with 1..32; anything
    else raises before a library is opened."""
    import pytest
    from gdn_state_codec import GdnStateCodecExperiment

    for initializer, iterations in (("quant_only", 0), ("quant_only", 32),
                                    ("exact_svd", 1), ("exact_svd", 32)):
        experiment = GdnStateCodecExperiment(initializer=initializer,
                                             boundary_power_iterations=iterations)
        assert experiment.initializer == initializer
    for initializer, iterations in (("exact_svd", 0), ("svd", 4), ("quant_only", 33),
                                    ("exact_svd", True), ("quant_only", -1)):
        with pytest.raises(RuntimeError, match="initializer|boundary_power_iterations"):
            GdnStateCodecExperiment(initializer=initializer,
                                    boundary_power_iterations=iterations)

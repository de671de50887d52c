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

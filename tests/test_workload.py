"""CPU checks of the synthetic decode workload's byte counts."""
import numpy as np



def test_unique_kv_bytes_counts_a_shared_row_once():
    """Without shared blocks the distinct-row count is the per-sequence count; with
    cfg4's prefix it is the union of the windows over the 15 shared blocks (the 16th
    is copied per sequence) plus each sequence's own rows."""
    from oxide_paged_kv.workload import CONFIGS, make_decode_step

    st = make_decode_step(CONFIGS[3], seed=5, batch=8)
    assert st.unique_kv_read_bytes() == st.kv_read_bytes()
    assert st.attn_unique_bytes() == st.attn_bytes()
    st = make_decode_step(CONFIGS[4], seed=5, batch=16)
    c = st.cfg
    L = st.context_lens.astype(np.int64)
    lo = np.maximum(L - 1 - c.window_left, 0)
    P = c.shared_prefix - c.block_size
    assert (L > P).all()
    rows = (P - lo.min()) + (L - np.maximum(lo, P)).sum()
    assert st.unique_kv_read_bytes() == 2 * rows * c.num_kv_heads * c.head_dim * 2
    assert st.attn_bytes() - st.attn_unique_bytes() == st.kv_read_bytes() - st.unique_kv_read_bytes()

"""oracle.pool spreads the paged oracle over processes: its outputs must be
the one-process functions' outputs bit for bit, and its key check must
notice a single flipped nibble."""

import numpy as np

from oracle import pack_int4, paged_decode_f64, paged_decode_ref, quantize_groups_ref
from oracle.pool import paged_oracle_all


def _workload():
    from flash_decode_int4.workloads import make_workload
    w = make_workload(batch=3, heads=4, head_dim=64, seq_lens=[300, 0, 700], seed=5,
                      q_heads=8)
    B, H, D = 3, 4, 64
    qr, sr, zr = quantize_groups_ref(w["k"], w["seq_lens"])
    kp = np.zeros((w["num_pages"], H, 16, D // 2), np.uint8)
    for b in range(B):
        n = int(w["seq_lens"][b])
        for lp in range((n + 15) // 16):
            r = min(16, n - lp * 16)
            kp[w["page_table"][b, lp], :, :r] = pack_int4(qr[b, :, lp * 16:lp * 16 + r])
    return w, dict(q=w["q"], kp=kp, v=w["v_pages"], s=sr, z=zr, pt=w["page_table"],
                   sl=w["seq_lens"], k=w["k"])


def test_pool_equals_one_process_and_checks_keys():
    w, arr = _workload()
    res = paged_oracle_all(arr, workers=3)
    args = (arr["q"], arr["kp"], arr["v"], arr["s"], arr["z"], arr["pt"], arr["sl"])
    np.testing.assert_array_equal(res["o32"], paged_decode_ref(*args))
    np.testing.assert_array_equal(res["o64"], paged_decode_f64(*args))
    assert res["key_mismatch"] == 0
    # One flipped bit in one stored row of sequence 2, kv-head 1.
    arr["kp"] = arr["kp"].copy()
    arr["kp"][w["page_table"][2, 5], 1, 3, 7] ^= 1
    assert paged_oracle_all(arr, workers=2, f64=False)["key_mismatch"] == 1
    # A changed zero-point of sequence 0, kv-head 3, group 2.
    arr["kp"][w["page_table"][2, 5], 1, 3, 7] ^= 1
    arr["z"] = arr["z"].copy()
    arr["z"][0, 3, 2, 11] = np.nextafter(arr["z"][0, 3, 2, 11], np.float32(np.inf))
    assert paged_oracle_all(arr, workers=2, f64=False)["key_mismatch"] == 1

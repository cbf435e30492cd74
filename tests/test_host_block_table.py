"""Device block-table deltas on the host (CPU).

``DeviceBlockTable.prepare_meta`` tells the pack kernel, per request state,
how many leading pages its table row already holds and which pages follow;
the kernel writes those after them.  Applying the same rule to a host copy
of the table after every step must reproduce every state's page list, whatever
the states went through: growth by ``extend``, replacement by a new list,
in-place rewrites of the first or last synced entry, an in-place edit flagged
with ``pages_changed``, release and re-acquire of slots, and table growth.
"""

import random

import numpy as np
import pytest
import torch

from mstar_amd.kv_store import DeviceBlockTable, KVRequestState


def _apply(table: np.ndarray, slots, npg, old, new) -> None:
    """What ``mi_pack`` does to the table with ``prepare_meta``'s output."""
    off = 0
    for s, n, o in zip(slots, npg, old):
        k = n - o
        table[s, o:n] = new[off:off + k]
        off += k
    assert off == len(new)


def _rows_match(bt: DeviceBlockTable, host: np.ndarray, states) -> None:
    for st in states:
        n = len(st.page_indices)
        assert list(host[st.slot, :n]) == st.page_indices


def test_delta_rules_reproduce_every_page_list():
    rng = random.Random(0)
    bt = DeviceBlockTable(64, torch.device("cpu"), max_slots=4)
    host = np.zeros((1024, 64), dtype=np.int32)
    states = [KVRequestState() for _ in range(12)]
    next_page = 0
    for step in range(300):
        for st in states:
            op = rng.random()
            n = len(st.page_indices)
            if op < 0.5 and n < 60:
                st.page_indices.extend(range(next_page, next_page + rng.randint(0, 3)))
            elif op < 0.6:
                st.page_indices = list(range(next_page, next_page + rng.randint(0, 20)))
            elif op < 0.7 and n:
                st.page_indices[-1] = next_page + 7  # last synced entry rewritten in place
            elif op < 0.75 and n:
                st.page_indices[0] = next_page + 9  # first entry rewritten in place
            elif op < 0.8 and n > 2:
                st.page_indices[n // 2] = next_page + 11  # middle entry: caller must flag it
                st.pages_changed()
            elif op < 0.85 and n > 1:
                st.page_indices[:] = st.page_indices[::-1]  # same object, same length, ends swapped
            elif op < 0.9:
                bt.release(st)
            next_page += 32
        subset = [st for st in states if rng.random() < 0.8]
        slots, npg, old, new = bt.prepare_meta(subset)
        if bt.max_slots > host.shape[0]:
            pytest.fail("table grew past the host copy")
        _apply(host, slots, npg, old, new)
        _rows_match(bt, host, subset)
    assert bt.max_slots >= 12  # grew from 4 rows


def test_unchanged_states_send_nothing():
    bt = DeviceBlockTable(16, torch.device("cpu"))
    st = KVRequestState(page_indices=[5, 6, 7])
    slots, npg, old, new = bt.prepare_meta([st])
    assert list(old) == [0] and list(new) == [5, 6, 7]
    slots, npg, old, new = bt.prepare_meta([st])
    assert list(old) == [3] and len(new) == 0
    st.page_indices.append(9)
    slots, npg, old, new = bt.prepare_meta([st])
    assert list(old) == [3] and list(new) == [9]
    st.page_indices[-1] = 10  # in place, same length: last entry differs -> full resend
    slots, npg, old, new = bt.prepare_meta([st])
    assert list(old) == [0] and list(new) == [5, 6, 7, 10]


def test_prepare_rejects_lists_longer_than_a_row():
    bt = DeviceBlockTable(4, torch.device("cpu"))
    with pytest.raises(ValueError):
        bt.prepare_meta([KVRequestState(page_indices=list(range(5)))])

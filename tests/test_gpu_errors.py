"""Misuse of the device ABI is refused on the host with a status and a message, before
any kernel is launched (the reference GPU backend panics on misuse, ops/attention.rs:28-36;
here the status reaches the caller)."""

from types import SimpleNamespace

import numpy as np
import pytest

from yaxus_amd._lib import YxError

pytestmark = pytest.mark.gpu
D = 128


def _meta(pos, slot, pt_off, pages):
    return SimpleNamespace(pos=np.array(pos, np.uint32), kv_slot=np.array(slot, np.uint32),
                           pt_off=np.array(pt_off, np.uint32), pages=np.array(pages, np.uint32))


@pytest.fixture
def kv(hip):
    kv = hip.new_kv(1, 8, 16, 2)
    yield kv
    kv.destroy()


def test_rejects_a_position_without_a_page_table_entry(hip, kv):
    hip.begin_pass(_meta([40], [3 * 16 + 8], [0], [3]))  # position 40 needs 3 pages
    with pytest.raises(YxError, match="page-table entry"):
        hip.attend(kv, 0, np.zeros((1, 4 * D), np.float32), 4)


def test_rejects_pages_beyond_the_arena(hip, kv):
    hip.begin_pass(_meta([0], [0], [0], [8]))
    with pytest.raises(YxError, match="beyond the arena"):
        hip.attend(kv, 0, np.zeros((1, 4 * D), np.float32), 4)


def test_rejects_head_counts_that_do_not_match(hip, kv):
    hip.begin_pass(_meta([0], [0], [0], [1]))
    with pytest.raises(YxError, match="multiple of hkv"):
        hip.attend(kv, 0, np.zeros((1, 3 * D), np.float32), 3)


def test_rejects_rows_of_one_sequence_that_are_not_consecutive(hip):
    with pytest.raises(YxError, match="not consecutive"):
        hip.begin_pass(_meta([0, 0, 1], [0, 16, 1], [0, 1, 0], [0, 1]))


def test_rejects_a_layer_beyond_the_arena(hip, kv):
    hip.begin_pass(_meta([0], [0], [0], [1]))
    with pytest.raises(YxError, match="layer"):
        hip.attend(kv, 3, np.zeros((1, 4 * D), np.float32), 4)


def test_the_context_still_works_after_an_error(hip, kv):
    hip.begin_pass(_meta([40], [3 * 16 + 8], [0], [3]))
    with pytest.raises(YxError):
        hip.attend(kv, 0, np.zeros((1, 4 * D), np.float32), 4)
    hip.begin_pass(_meta([0], [16], [0], [1]))
    k = np.ones((1, 2, D), np.float32)
    hip.append(kv, 0, k, k * 2)
    out = hip.attend(kv, 0, np.zeros((1, 4 * D), np.float32), 4)
    assert np.all(out[0, :D] == 2.0)  # one key: the output is its value


def test_a_graph_is_refused_after_the_pass_changes(hip, kv):
    """A captured graph points at the pass's work list; a new pass frees it, so the graph
    is refused instead of replayed."""
    q = hip.tensor((1, 4 * D))
    out = hip.tensor((1, 4 * D))
    hip.begin_pass(_meta([5], [5], [0], [1]))
    hip.attend(kv, 0, q, 4, out=out)
    hip.graph_begin()
    hip.attend(kv, 0, q, 4, out=out)
    hip.graph_end()
    hip.graph_launch()
    hip.sync()
    hip.set_option("attn_target_waves", 0)  # drops the work lists
    with pytest.raises(YxError, match="capture it again"):
        hip.graph_launch()
    hip.attend(kv, 0, q, 4, out=out)
    hip.graph_begin()
    hip.attend(kv, 0, q, 4, out=out)
    hip.graph_end()
    hip.graph_launch()
    hip.begin_pass(_meta([6], [6], [0], [1]))
    with pytest.raises(YxError, match="capture it again"):
        hip.graph_launch()
    hip.sync()
    for t in (q, out):
        t.free()


def test_rejects_null_device_buffers(hip, kv):
    """Null q, out, k or v on the device-pointer entry points is refused on the host
    (a kernel given a null buffer would fault the GPU instead)."""
    from yaxus_amd._lib import YX_OK

    hip.begin_pass(_meta([5], [5], [0], [1]))
    out = hip.tensor((1, 4 * D))
    q = hip.tensor((1, 4 * D))
    kk = hip.tensor((1, 2 * D))
    scale = 1.0 / np.sqrt(D)
    L = hip.L
    assert L.yx_attention_dev(hip.ctx, kv.h, 0, None, out.ptr, 4, 2, 0, scale) != YX_OK
    assert L.yx_attention_dev(hip.ctx, kv.h, 0, q.ptr, None, 4, 2, 0, scale) != YX_OK
    assert L.yx_attention_append_dev(hip.ctx, kv.h, 0, kk.ptr, None, q.ptr, out.ptr, 4, 2, 0,
                                     scale) != YX_OK
    assert L.yx_kv_append_dev(hip.ctx, kv.h, 0, None, kk.ptr) != YX_OK
    hip.attend(kv, 0, q, 4, out=out)  # the context still works
    hip.sync()
    for t in (out, q, kk):
        t.free()


def test_python_mirror_rejects_short_device_tensors(hip, kv):
    """The C ABI takes plain pointers and cannot see a buffer's size; the Python mirror
    checks device tensors against the pass's rows and the arena's heads (here K/V sized
    for one KV head against an arena of two) before any launch."""
    hip.begin_pass(_meta([0, 1], [0, 1], [0, 0], [0]))
    q, out = hip.tensor((2, 4 * D)), hip.tensor((2, 4 * D))
    k, v = hip.tensor((2, D)), hip.tensor((2, D))
    try:
        with pytest.raises(ValueError, match="k: device tensor"):
            hip.attend_append(kv, 0, k, v, q, 4, out=out)
        with pytest.raises(ValueError, match="k: device tensor"):
            hip.append(kv, 0, k, v)
        with pytest.raises(ValueError, match="q: device tensor"):
            hip.attend(kv, 0, q, 8, out=out)
    finally:
        for t in (q, out, k, v):
            t.free()

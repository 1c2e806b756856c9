"""Host logic (no GPU): objects that borrow layer handles are rebuilt when a layer's handle is re-created.

The dense GatedKAN block and the multi-layer chain keep raw ``kans_layer`` pointers.  Changing a layer's
dtype destroys its handle and creates a new one, which the allocator is free to place at the old address.
These tests run the Python layer logic against a stand-in library whose allocator hands back the most
recently freed address, and check that the block / chain is re-created on the new handles (a cache keyed
on addresses would keep the destroyed ones and the old dtype).
"""
import ctypes

import numpy as np
import pytest


class FakeLib:
    """The library calls the layer, chain and dense-block Python code makes, with LIFO address reuse."""

    def __init__(self):
        self.free = []
        self.next = 0x1000
        self.live = {}            # address -> dtype of live kans_layer handles
        self.blocks = {}          # dense block / chain address -> tuple of layer addresses
        self.block_creates = 0
        self.chain_creates = 0
        self.forwards = []        # (kind, object address) per forward call

    def _alloc(self):
        if self.free:
            return self.free.pop()
        self.next += 0x100
        return self.next

    @staticmethod
    def _set(ref, v):
        ref._obj.value = v

    def kans_last_error(self):
        return b""

    def kans_layer_create(self, basis, dt, d_in, d_out, K, hb, hbias, ref):
        a = self._alloc()
        self.live[a] = dt
        self._set(ref, a)
        return 0

    def kans_layer_destroy(self, h):
        a = h.value if isinstance(h, ctypes.c_void_p) else h
        del self.live[a]
        self.free.append(a)
        return 0

    def kans_layer_load_weights(self, *a):
        return 0

    kans_layer_load_weights_f32 = kans_layer_load_weights

    def kans_layer_set_tiling(self, *a):
        return 0

    kans_layer_set_wave_groups = kans_layer_set_tiling

    def kans_gated_dense_create(self, g, u, d, ref):
        for h in (g, u, d):
            assert h in self.live, "block created on a destroyed layer handle"
        a = self._alloc()
        self.blocks[a] = (g, u, d)
        self.block_creates += 1
        self._set(ref, a)
        return 0

    def kans_gated_dense_destroy(self, h):
        a = h.value if isinstance(h, ctypes.c_void_p) else h
        del self.blocks[a]
        self.free.append(a)
        return 0

    def kans_gated_dense_forward_host(self, blk, x, x_dt, y, B):
        a = blk.value if isinstance(blk, ctypes.c_void_p) else blk
        for h in self.blocks[a]:
            assert h in self.live, "forward through a destroyed layer handle"
        self.forwards.append(("dense", a))
        return 0

    def kans_chain_create(self, arr, n, ref):
        hs = tuple(arr[i] for i in range(n))
        for h in hs:
            assert h in self.live, "chain created on a destroyed layer handle"
        a = self._alloc()
        self.blocks[a] = hs
        self.chain_creates += 1
        self._set(ref, a)
        return 0

    kans_chain_destroy = kans_gated_dense_destroy

    def kans_chain_forward_host_ex(self, chain, x, x_dt, y, B):
        a = chain.value if isinstance(chain, ctypes.c_void_p) else chain
        for h in self.blocks[a]:
            assert h in self.live, "forward through a destroyed layer handle"
        self.forwards.append(("chain", a))
        return 0


@pytest.fixture
def fake(monkeypatch):
    from metal_kans import device
    lib = FakeLib()
    monkeypatch.setattr(device, "get_metal_bridge", lambda: lib)
    monkeypatch.setattr(device, "load_library", lambda *a, **k: lib)
    return lib


def test_gated_dense_block_rebuilt_after_dtype_change(fake):
    import metal_kans as mk
    np.random.seed(0)
    blk = mk.GatedKAN(d_model=8, d_ffn=16, degree=3)
    x = np.random.uniform(-1, 1, (5, 8)).astype(np.float32)
    blk(x)
    assert fake.block_creates == 1
    first = blk._dense_block.value
    old_handles = set(fake.blocks[first])
    for k in (blk.gate_kan, blk.up_kan, blk.down_kan):
        k.half()
    blk(x)
    # the fp16 handles reuse the fp32 handles' addresses (LIFO allocator) ...
    assert set(fake.blocks[blk._dense_block.value]) == old_handles
    # ... but the block was re-created on them, once
    assert fake.block_creates == 2
    assert all(fake.live[h] == 1 for h in fake.blocks[blk._dense_block.value])
    blk(x)
    assert fake.block_creates == 2          # unchanged layers reuse the block


def test_gated_forward_clears_sublayer_inputs(fake):
    import metal_kans as mk
    np.random.seed(1)
    blk = mk.GatedKAN(d_model=8, d_ffn=16, degree=3)
    blk.down_kan._saved_x = np.zeros((2, 16), np.float32)     # as after a direct call to the layer
    blk(np.random.uniform(-1, 1, (3, 8)).astype(np.float32))
    for k in (blk.gate_kan, blk.up_kan, blk.down_kan):
        assert k._saved_x is None
    with pytest.raises(RuntimeError, match="before forward"):
        blk.down_kan.backward(np.zeros((3, 8), np.float32))


def test_chain_rebuilt_after_dtype_change(fake):
    import metal_kans as mk
    np.random.seed(2)
    net = mk.MetalKAN([8, 12, 4], basis_type="cheby", degree=3)
    x = np.random.uniform(-1, 1, (6, 8)).astype(np.float32)
    net(x)
    assert fake.chain_creates == 1
    net.half()
    net(x)
    assert fake.chain_creates == 2
    assert all(fake.live[h] == 1 for h in fake.blocks[net._chain.value])
    net(x)
    assert fake.chain_creates == 2

"""Host-only driver of the native slot cache (sluice_layer_* with no device
map): runs the same bookkeeping the device gap runs, so the C++ state
machine can be compared with the oracle and the golden vectors on the CPU."""

import ctypes

from sluice_amd import _lib


class NativeCache:
    def __init__(self, E, local_n, slots, protect_frac=0.5, local_of=None, lfu=False,
                 counts=False):
        self.lib = _lib.load()
        self.E, self.local_n = E, local_n
        self.S = min(slots, local_n)
        frac = min(max(float(protect_frac), 0.0), 0.9)
        cap = max(min(int(self.S * frac), self.S - 1), 0)
        lof = _lib.int32_array(local_of if local_of is not None else range(E))
        h = ctypes.c_void_p()
        _lib.check(self.lib.sluice_layer_create(E, local_n, self.S, cap, lof, None,
                                                ctypes.byref(h)), "sluice_layer_create")
        self.h = h.value
        self._streams = (ctypes.c_int32 * (2 * max(self.S, 1)))()
        if lfu or counts:
            _lib.check(self.lib.sluice_layer_set_policy(self.h, int(lfu), int(counts)),
                       "sluice_layer_set_policy")

    def policy(self):
        freq = (ctypes.c_int64 * self.local_n)()
        dec = (ctypes.c_int64 * self.E)()
        scan = (ctypes.c_int64 * self.E)()
        st = (ctypes.c_int64 * 3)()
        _lib.check(self.lib.sluice_layer_policy_state(self.h, freq, dec, scan, st), "policy")
        return {"freq": [[l, f] for l, f in enumerate(freq) if f],
                "counts_decode": list(dec), "counts_scan": list(scan),
                "steps_small": st[0], "steps_scan": st[1], "lfu_steps": st[2]}

    def step_stats(self):
        """{"small"|"scan": {steps, hits, misses, waves}} of real classic steps."""
        out = (ctypes.c_int64 * 8)()
        _lib.check(self.lib.sluice_layer_step_stats(self.h, out), "step_stats")
        keys = ("steps", "hits", "misses", "waves")
        return {kind: {k: int(out[4 * i + j]) for j, k in enumerate(keys)}
                for i, kind in enumerate(("small", "scan"))}

    def __del__(self):
        if getattr(self, "h", None):
            self.lib.sluice_layer_destroy(self.h)
            self.h = None

    def pin(self, local, debit=True):
        s = ctypes.c_int()
        rc = self.lib.sluice_layer_pin(self.h, local, int(debit), ctypes.byref(s))
        return None if rc else s.value

    def unfill(self, slot):
        """True when the slot's expert left the cache."""
        rc = self.lib.sluice_layer_unfill(self.h, slot)
        if rc == _lib.SLUICE_E_STATE:
            return False
        _lib.check(rc, "sluice_layer_unfill")
        return True

    def gap(self, ids, fast_hit=False):
        """Returns (streams, overflow)."""
        arr = _lib.int32_array(ids)
        n = ctypes.c_int()
        mw = ctypes.c_int()
        rc = self.lib.sluice_layer_gap_host(self.h, arr, len(ids), int(fast_hit), self._streams,
                                            self.S, ctypes.byref(n), ctypes.byref(mw))
        streams = [[self._streams[2 * i], self._streams[2 * i + 1]] for i in range(n.value)]
        if rc == _lib.SLUICE_E_OVERFLOW:
            return streams, True
        _lib.check(rc, "sluice_layer_gap_host")
        return streams, False

    def classic(self, ids, T, nd=None, ndec=None, real_step=True, spec_tokens=0):
        """One classic step on host ids; returns the waves as the oracle does
        ([{"pairs": [(g, slot)], "streams": [(local, slot)]}])."""
        arr = _lib.int32_array(ids)
        nw = ctypes.c_int()
        _lib.check(self.lib.sluice_layer_classic_host(
            self.h, arr, len(ids), T, -1 if nd is None else nd, -1 if ndec is None else ndec,
            int(real_step), spec_tokens, ctypes.byref(nw)), "sluice_layer_classic_host")
        waves, _ = read_plan(self.lib, self.h)
        assert len(waves) == nw.value
        return waves

    def state(self):
        S, L = self.S, self.local_n
        slot_of = (ctypes.c_int32 * L)()
        eis = (ctypes.c_int32 * S)()
        prob = (ctypes.c_int32 * S)()
        prot = (ctypes.c_int32 * S)()
        free = (ctypes.c_int32 * S)()
        n_prob, n_prot, n_free = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        ctr = (ctypes.c_int64 * 8)()
        m = (ctypes.c_int32 * self.E)()
        _lib.check(self.lib.sluice_layer_state(self.h, slot_of, eis, prob, ctypes.byref(n_prob),
                                               prot, ctypes.byref(n_prot), free,
                                               ctypes.byref(n_free), ctr), "state")
        _lib.check(self.lib.sluice_layer_standing_map(self.h, m), "standing_map")
        return {
            "slot_of": list(slot_of),
            "expert_in_slot": list(eis),
            "probation": list(prob)[: n_prob.value],
            "protected": list(prot)[: n_prot.value],
            "free_slots": list(free)[: n_free.value],
            "standing_map": list(m),
            "map_is_standing": bool(ctr[6]),
            "protected_cap": int(ctr[7]),
            "counters": {"gaps": ctr[0], "misses": ctr[1], "fast_hits": ctr[2],
                         "map_writes": ctr[3]},
        }


def read_plan(lib, handle):
    """The layer's last classic plan: (waves, pipelined)."""
    n = ctypes.c_int()
    _lib.check(lib.sluice_layer_classic_plan_read(handle, None, 0, ctypes.byref(n), None),
               "sluice_layer_classic_plan_read")
    buf = (ctypes.c_int32 * max(n.value, 1))()
    _lib.check(lib.sluice_layer_classic_plan_read(handle, buf, n.value, ctypes.byref(n), None),
               "sluice_layer_classic_plan_read")
    v = list(buf)[: n.value]
    nw, pipelined, i = v[0], bool(v[1]), 2
    waves = []
    for _ in range(nw):
        npairs = v[i]
        pairs = [(v[i + 1 + 2 * j], v[i + 2 + 2 * j]) for j in range(npairs)]
        i += 1 + 2 * npairs
        ns = v[i]
        streams = [(v[i + 1 + 2 * j], v[i + 2 + 2 * j]) for j in range(ns)]
        i += 1 + 2 * ns
        waves.append({"pairs": pairs, "streams": streams})
    assert i == len(v)
    return waves, pipelined

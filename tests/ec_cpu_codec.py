"""Oracle-backed slice codec: a test double of GpuSliceCodec for CPU tests
of the erasure-coded checkpoint manager (exchange, placement, files,
failure handling).  Same slice format: slice p is the concatenation over
stripes of codeword position p, zero-padded units of unit_bytes.  Test
infrastructure: the product's codec is the GPU one."""
import numpy as np
import torch

import oracle

GENERATOR_ID = "gf256-0x11d-cauchy1"


def _tensor_bytes(t):
    return t.detach().contiguous().reshape(-1).view(torch.uint8).numpy()


class _Staged:
    """What GpuSliceCodec.snapshot returns, already complete (or failing
    when its result is asked for, as a staging error would)."""

    def __init__(self, meta, slices, error=None):
        self._meta, self._slices, self._error = meta, slices, error

    def done(self):
        return True

    def result(self, timeout=None):
        if self._error is not None:
            raise self._error
        return self._meta, self._slices


class OracleSliceCodec:
    """fail: encode and snapshot raise; fail_late: snapshot returns, its
    result() raises (a failure during background staging)."""

    def __init__(self, k, m, unit_bytes, fail=False, fail_late=False):
        self.k, self.m, self.unit_bytes, self.fail = k, m, unit_bytes, fail
        self.fail_late = fail_late
        self.changed_log = []   # the changed_tensors of each call (None: a full save)

    def snapshot(self, tensors, changed_tensors=None):
        meta, slices = self.encode(tensors, changed_tensors)
        err = RuntimeError("injected staging failure") if self.fail_late else None
        return _Staged(meta, slices, err)

    def _units(self, bufs):
        U = self.unit_bytes
        units, lens = [], []
        for b in bufs:
            for o in range(0, b.size, U):
                units.append(b[o: o + U])
                lens.append(min(U, b.size - o))
        return units, lens

    def encode(self, tensors, changed_tensors=None):
        """The full encode, also when changed_tensors names the tensors that
        changed (the slices are the same)."""
        self.changed_log.append(None if changed_tensors is None else list(changed_tensors))
        if self.fail:
            raise RuntimeError("injected encode failure")
        k, m, U = self.k, self.m, self.unit_bytes
        units, lens = self._units([_tensor_bytes(t) for t in tensors])
        S = max(1, -(-len(units) // k))
        grid = [[units[s * k + j] if s * k + j < len(units) else None for j in range(k)]
                for s in range(S)]
        glen = np.array([[lens[s * k + j] if s * k + j < len(units) else 0 for j in range(k)]
                         for s in range(S)], np.uint32)
        parity = oracle.encode_batched(oracle.cauchy(k, m), grid, glen, U)
        slices = []
        for p in range(k):
            sl = np.zeros((S, U), np.uint8)
            for s in range(S):
                if grid[s][p] is not None:
                    sl[s, : grid[s][p].size] = grid[s][p]
            slices.append(sl.reshape(-1))
        slices += [np.ascontiguousarray(parity[:, i]).reshape(-1) for i in range(m)]
        meta = {"k": k, "m": m, "unit_bytes": U, "n_stripes": S, "n_units": len(units),
                "tensors": [{"dtype": str(t.dtype).replace("torch.", ""), "shape": list(t.shape),
                             "nbytes": t.numel() * t.element_size()} for t in tensors],
                "generator": GENERATOR_ID}
        return meta, slices

    def decode(self, meta, slices, device):
        k, m, U, S = meta["k"], meta["m"], meta["unit_bytes"], meta["n_stripes"]
        have = dict(slices)
        lost = [p for p in range(k + m) if p not in have]
        if any(p < k for p in lost):
            surv, rows = oracle.decode_matrix(oracle.cauchy(k, m), k, m, lost)
            rec = oracle.rs_encode(rows, [have[s] for s in surv])
            have.update(dict(zip(lost, rec)))
        stream = np.stack([have[p].reshape(S, U) for p in range(k)], axis=1).reshape(-1)
        out, unit_idx = [], 0
        for tm in meta["tensors"]:
            t = torch.empty(tm["shape"], dtype=getattr(torch, tm["dtype"]))
            flat = t.reshape(-1).view(torch.uint8).numpy()
            for o in range(0, flat.size, U):
                n = min(U, flat.size - o)
                flat[o: o + n] = stream[unit_idx * U: unit_idx * U + n]
                unit_idx += 1
            out.append(t.to(device))
        return out

"""Test double of MCoreTensorAwareStateDict's tensor protocol
(megatron/core/dist_checkpointing/tensor_aware_state_dict.py:154-232):
``tensors`` is an iterator over the shard tensors, ``pop_tensors`` hollows
the object and returns them, ``insert_tensors`` puts them back, and
``to_state_dict`` needs the tensors in place.  It is pickled by the
checkpoint manager while hollow, so it lives in an importable module."""


class FakeTensorAwareStateDict:
    def __init__(self, tensors, common, names):
        self.common = common
        self.names = list(names)
        self._data = list(tensors)
        self._is_hollow = False

    @property
    def is_hollow(self):
        return self._is_hollow

    @property
    def tensors(self):
        assert not self._is_hollow
        return map(lambda t: t, self._data)

    def pop_tensors(self):
        assert not self._is_hollow
        out, self._data = self._data, [None] * len(self._data)
        self._is_hollow = True
        return out

    def insert_tensors(self, tensors):
        assert self._is_hollow
        tensors = list(tensors)
        assert len(tensors) == len(self._data)
        self._data = tensors
        self._is_hollow = False

    def to_state_dict(self):
        assert not self._is_hollow
        return {"common": self.common, **dict(zip(self.names, self._data))}

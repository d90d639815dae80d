# SPDX-FileCopyrightText: Copyright contributors to the spconv-Triton project
# SPDX-FileCopyrightText: Derived from spconv, Copyright 2021 Yan Yan and contributors
# SPDX-License-Identifier: Apache-2.0
# The public names, signatures and error messages in this file follow spconv-Triton's
# API (Apache-2.0); the implementation is this package's own.
"""Device hash table, a drop-in for ``spconv_triton.pytorch.hash.HashTable``
(reference ``spconv_triton/pytorch/hash.py:15-110``).

The reference keeps sorted key/value arrays and re-sorts them on every
insert; here the table is an open-addressing hash in one device buffer
(csrc/sp_hashtable.hip) with the same observable behaviour: the last value
given for a key wins, ``query`` returns (values, is_empty), and ``items`` /
``assign_arange_`` enumerate the entries in ascending key order.  Keys are
int32 or int64 (the int64 key INT64_MAX is reserved); values are int32,
int64, float32 or float64.  GPU tables only: this package has no CPU path.
"""

from __future__ import annotations

import ctypes

import torch

from spconv_triton.pytorch._impl import _lib

_VKIND = {torch.int32: 0, torch.int64: 1, torch.float32: 2, torch.float64: 3}


class HashTable:
    def __init__(self, device: torch.device, key_dtype: torch.dtype, value_dtype: torch.dtype,
                 max_size: int = -1):
        if key_dtype not in (torch.int32, torch.int64):
            raise AssertionError
        if device.type != "cpu" and max_size <= 0:
            raise AssertionError("you must provide max_size for fixed-size cuda hash table, "
                                 "usually *2 of num of keys")
        if device.type != "cuda":
            raise NotImplementedError("spconv_triton's HashTable lives in GPU memory")
        if value_dtype not in _VKIND:
            raise NotImplementedError(f"HashTable values of dtype {value_dtype}")
        self.device = device
        self.key_dtype = key_dtype
        self.value_dtype = value_dtype
        self.max_size = max_size
        cap = 1024
        while cap < 2 * max_size:
            cap *= 2
        self._cap = cap
        self._key64 = int(key_dtype == torch.int64)
        self._vkind = _VKIND[value_dtype]
        self._epoch = 0
        self._count = 0
        L = _lib.lib()
        self._table = torch.empty(L.sp_hash_table_bytes(cap), dtype=torch.uint8, device=device)
        _lib.check(L.sp_hash_clear(_lib.ptr(self._table), cap, self._stream()), "sp_hash_clear")

    def _stream(self):
        return _lib.stream_of(self._table.device)

    def _keys(self, keys):
        return keys.to(self.device).to(self.key_dtype).reshape(-1).contiguous()

    def _values(self, values, n):
        return values.to(self.device).to(self.value_dtype).reshape(-1)[:n].contiguous()

    def _ws(self, n):
        return _lib.workspace(_lib.lib().sp_hash_workspace_size(self._cap, n), self.device)

    def insert(self, keys: torch.Tensor, values: torch.Tensor | None = None):
        keys = self._keys(keys)
        n = keys.numel()
        vals = None if values is None else self._values(values, n)
        self._epoch += 1
        count = ctypes.c_int64(0)
        ws = self._ws(n)
        rc = _lib.lib().sp_hash_insert(
            _lib.ptr(self._table), self._cap, _lib.ptr(keys), self._key64, _lib.ptr(vals),
            self._vkind, n, self._epoch, ctypes.byref(count), _lib.ptr(ws), ws.numel(),
            self._stream())
        if rc == _lib.SP_ERR_HASH_FULL:
            raise AssertionError("hash table full")
        _lib.check(rc, "sp_hash_insert")
        self._count = int(count.value)
        if self.max_size > 0 and self._count > self.max_size:
            raise AssertionError("hash table full")

    def query(self, keys: torch.Tensor, values: torch.Tensor | None = None):
        keys = self._keys(keys)
        n = keys.numel()
        out_v = torch.zeros(n, dtype=self.value_dtype, device=self.device)
        is_empty = torch.ones(n, dtype=torch.bool, device=self.device)
        if n:
            _lib.check(_lib.lib().sp_hash_query(
                _lib.ptr(self._table), self._cap, _lib.ptr(keys), self._key64, self._vkind, n,
                _lib.ptr(out_v), _lib.ptr(is_empty), self._stream()), "sp_hash_query")
        if values is not None:
            values.reshape(-1)[:n].copy_(out_v)
        return out_v, is_empty

    def insert_exist_keys(self, keys: torch.Tensor, values: torch.Tensor):
        keys = self._keys(keys)
        n = keys.numel()
        vals = self._values(values, n)
        found = torch.zeros(n, dtype=torch.bool, device=self.device)
        if n:
            self._epoch += 1
            ws = self._ws(n)
            _lib.check(_lib.lib().sp_hash_insert_existing(
                _lib.ptr(self._table), self._cap, _lib.ptr(keys), self._key64, _lib.ptr(vals),
                self._vkind, n, self._epoch, _lib.ptr(found), _lib.ptr(ws), ws.numel(),
                self._stream()), "sp_hash_insert_existing")
        return found

    def _count_tensor(self, n):
        dtype = torch.int32 if self.key_dtype == torch.int32 else torch.int64
        return torch.tensor([n], dtype=dtype, device=self.device)

    def assign_arange_(self):
        ws = self._ws(0)
        _lib.check(_lib.lib().sp_hash_items(
            _lib.ptr(self._table), self._cap, self._key64, self._vkind, 0, None, None, 1,
            _lib.ptr(ws), ws.numel(), self._stream()), "sp_hash_items")
        return self._count_tensor(self._count)

    def items(self, max_size: int = -1):
        """(keys, values, count): buffers of max_size entries (the table's
        max_size if -1), the first `count` holding the stored pairs in
        ascending key order."""
        if max_size == -1:
            max_size = self.max_size
        n = min(self._count, max_size)
        keys = torch.zeros([max_size], dtype=self.key_dtype, device=self.device)
        values = torch.zeros([max_size], dtype=self.value_dtype, device=self.device)
        if n:
            ws = self._ws(0)
            _lib.check(_lib.lib().sp_hash_items(
                _lib.ptr(self._table), self._cap, self._key64, self._vkind, n, _lib.ptr(keys),
                _lib.ptr(values), 0, _lib.ptr(ws), ws.numel(), self._stream()), "sp_hash_items")
        return keys, values, self._count_tensor(n)

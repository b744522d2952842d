"""Allocator restatement (TEST INFRASTRUCTURE ONLY): the reference
scheduler's KV block bookkeeping, line for line in meaning:

- free list: a vector initialised to [n-1, ..., 1, 0]   (src/sched.rs:515)
- take_blocks(n): split_off(len - n) -> the last n in vector order, refs = 1
                                                         (src/sched.rs:801-807)
- unref_blocks: refs -= 1; at 0 push back on the end    (src/sched.rs:809-817)
- sharing a cached prefix adds a reference per block    (src/sched.rs:758-760,
                                                         1054-1056)
Reference counts are u16 (src/sched.rs:464).
"""


class BlockPool:
    def __init__(self, n):
        self.free = list(range(n - 1, -1, -1))
        self.refs = [0] * n

    def take(self, n):
        if n > len(self.free):
            raise ValueError("not enough free blocks")
        out = self.free[len(self.free) - n:]
        del self.free[len(self.free) - n:]
        for b in out:
            self.refs[b] = 1
        return out

    def unref(self, blocks):
        for b in blocks:
            if self.refs[b] == 0:
                raise ValueError("refcount underflow")
            self.refs[b] -= 1
            if self.refs[b] == 0:
                self.free.append(b)

    def ref(self, blocks):
        for b in blocks:
            if self.refs[b] == 0 or self.refs[b] >= 0xFFFF:
                raise ValueError("bad ref")
            self.refs[b] += 1

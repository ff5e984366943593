//go:build linux

package enchip

import (
	"errors"
	"unsafe"

	"github.com/townsendmerino/aikit/ann"
)

// annBackend serves ann.Backend (ann/backend.go:16-55) from the same context: an index is a
// registered weight, its scores the bias-free W8A8 linear, TopKBatch the device top-k.
type annBackend struct{ b *Backend }

func (a annBackend) Name() string { return "hip" }

func (a annBackend) NewI8Index(bq []int8, scales []float32, n, dim int) (ann.I8Index, error) {
	a.b.mu.Lock()
	defer a.b.mu.Unlock()
	var h uint64
	var err error
	pinned(func() {
		if rc := cWeightRegister(a.b.ctx, unsafe.Pointer(&bq[0]), unsafe.Pointer(&scales[0]), int64(n), int64(dim), &h); rc != statusOK {
			err = errors.New(cLastError(a.b.ctx))
		}
	})
	if err != nil {
		return nil, err
	}
	return &i8Index{b: a.b, h: h, n: n, dim: dim}, nil
}

type i8Index struct {
	b      *Backend
	h      uint64
	n, dim int
}

// Score: dst[j] = W8A8(q, row j), as linalg.MatmulBTW8A8 computes it.
func (x *i8Index) Score(q, dst []float32) error {
	x.b.mu.Lock()
	defer x.b.mu.Unlock()
	var err error
	pinned(func() {
		if rc := cLinear(x.b.ctx, x.h, unsafe.Pointer(&q[0]), 1, nil, actNone, unsafe.Pointer(&dst[0]), nil); rc != statusOK {
			err = errors.New(cLastError(x.b.ctx))
		}
	})
	return err
}

// ScoreBatch (ann.I8BatchIndex): one W8A8 GEMM over all M queries.
func (x *i8Index) ScoreBatch(queries [][]float32, dst []float32) error {
	a := make([]float32, 0, len(queries)*x.dim)
	for _, q := range queries {
		a = append(a, q...)
	}
	x.b.mu.Lock()
	defer x.b.mu.Unlock()
	var err error
	pinned(func() {
		if rc := cLinear(x.b.ctx, x.h, unsafe.Pointer(&a[0]), int64(len(queries)), nil, actNone, unsafe.Pointer(&dst[0]), nil); rc != statusOK {
			err = errors.New(cLastError(x.b.ctx))
		}
	})
	return err
}

// TopKBatch (ann.I8TopKIndex): each query's k best hits, selected on the device.
// enchip_ann_topk pads a query with fewer than k non-NaN scores with index -1.
func (x *i8Index) TopKBatch(queries [][]float32, k int) ([][]ann.Hit, error) {
	a := make([]float32, 0, len(queries)*x.dim)
	for _, q := range queries {
		a = append(a, q...)
	}
	idx := make([]int32, len(queries)*k)
	sc := make([]float32, len(queries)*k)
	var err error
	x.b.mu.Lock()
	pinned(func() {
		if rc := cAnnTopK(x.b.ctx, x.h, unsafe.Pointer(&a[0]), int64(len(queries)), int64(k),
			unsafe.Pointer(&idx[0]), unsafe.Pointer(&sc[0])); rc != statusOK {
			err = errors.New(cLastError(x.b.ctx))
		}
	})
	x.b.mu.Unlock()
	if err != nil {
		return nil, err
	}
	out := make([][]ann.Hit, len(queries))
	for m := range queries {
		for i := 0; i < k && idx[m*k+i] >= 0; i++ {
			out[m] = append(out[m], ann.Hit{Index: int(idx[m*k+i]), Score: float64(sc[m*k+i])})
		}
	}
	return out, nil
}

func (x *i8Index) Close() error {
	x.b.mu.Lock()
	defer x.b.mu.Unlock()
	cWeightRelease(x.b.ctx, x.h)
	return nil
}

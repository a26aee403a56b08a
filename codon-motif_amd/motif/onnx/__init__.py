'''The static-graph step boundary of the model (`motif.onnx.step`).

Exporting to ONNX and running under ONNX Runtime are not part of this package; the
step module is: a decode / prefill step as a pure function of flat cache tensors,
the I/O a captured graph or a serving loop binds to.
'''

"""Drop-in MI355X implementation of ``ffnmem.memory`` (the route n-gram memory layer)."""

class KVConnectorBase_v1:
    def __init__(self, *args, **kwargs):
        self.base_args = (args, kwargs)
